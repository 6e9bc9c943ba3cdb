/*
 * lngram_hip.h -- C ABI of the MI355X (gfx950) route n-gram memory hot path.
 *
 * Conventions (every entry point):
 *   - Tensors are caller-owned device buffers, row-major and contiguous.
 *   - Calls are ordered on `stream` (a hipStream_t passed as void*), keep no
 *     pointer to a caller's buffer after return, and return 0 or a negative LNG_E_*.
 *   - Device memory is the caller's: scratch comes in as a workspace argument.
 *     Two kinds of host-side state are kept per process, each made once and
 *     guarded by a mutex, so calls stay reentrant from any host thread:
 *       * lng_drafter_tree_levels caches its resident grid size per device;
 *       * lng_ssm_scan_static uses a static device array per GPU (its own
 *         comment gives the limit), located once per device.
 *   - lng_last_error() returns a thread-local message for the last failure.
 *   - dtype codes: LNG_F32, LNG_BF16, LNG_F16, LNG_U8, LNG_I32, LNG_I64.
 *
 * Each declaration names the reference interface (file:line in the reference
 * repository) whose computation it replaces.
 */
#ifndef LNGRAM_HIP_H
#define LNGRAM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { LNG_F32 = 0, LNG_BF16 = 1, LNG_F16 = 2, LNG_U8 = 3, LNG_I32 = 4, LNG_I64 = 5 };
enum {
  LNG_OK = 0,
  LNG_E_ARG = -1,      /* bad shape / argument */
  LNG_E_DTYPE = -2,    /* unsupported dtype combination */
  LNG_E_HIP = -3,      /* HIP launch / runtime error */
  LNG_E_RANGE = -4     /* value out of range (token id, index) */
};

int lng_abi_version(void);
const char* lng_last_error(void);

/* ---------------------------------------------------------------- K1: router */
/* y[M,N] (fp32) = x[M,K] . w[N,K]^T.  LngramMemory.route_logits
 * (ffnmem/memory/wrapper.py:98-101).  bf16 x bf16 runs on MFMA with fp32
 * accumulation (products of bf16 values are exact in fp32); f32 x f32 runs in
 * fp32 FMA.  If `codes` is non-null the epilogue also sign-packs every `bits`
 * consecutive channels into route codes (lngram_v2.py:74-89, :1012-1017) of
 * dtype codes_dtype (LNG_U8 or LNG_I32), shape [M, N/bits]; `logits` may be null. */
int lng_router_codes(const void* x, int x_dtype, const void* w, int w_dtype, int64_t M, int64_t K,
                     int64_t N, int32_t bits, float* logits, void* codes, int codes_dtype, void* stream);

/* codes[M, C/bits] = pack(logits[M, C] > 0).  quantize_route_logits
 * (lngram_v2.py:1012-1017 -> pack_bits_to_route_codes :74-89). */
int lng_pack_route_codes(const float* logits, int64_t M, int64_t C, int32_t bits, void* codes,
                         int codes_dtype, void* stream);

/* out[B*T, 2d+N] = concat(RMSNorm(E[x_{t-1}] or start; prev_w), RMSNorm(E[x_t]; cur_w)[, s_t])
 * in `dtype` (bf16 or fp32): TokenRouterFeatures.forward (ffnmem/memory/router.py:50-59) with
 * model.RMSNorm's rounding (ffnmem/model.py:39-48: normalise in fp32, round, times the weight).
 * Rows: token_ids != null -> emb is the [vocab, d] table and row t is emb[token_ids[t]] (an id
 * outside [0, vocab) reads a zero row); token_ids == null -> emb is [B*T, d] (E[x] already
 * gathered).  ssm_state [B*T, N] fp32 (embed2_ssm) or null with N = 0.  d * elem and
 * (2d + N) * elem must be multiples of 16 bytes, d <= 4096 (bf16) / 2048 (fp32). */
int lng_router_features(const void* emb, int dtype, const int64_t* token_ids, int64_t vocab, int64_t B, int64_t T,
                        int32_t d, const void* start, const void* prev_w, const void* cur_w, float eps,
                        const float* ssm_state, int32_t N, void* out, void* stream);

/* The token router's tables (bf16): fprev [vocab+2, d] = RMSNorm(E[v]; prev_w) for every row v,
 * then RMSNorm(start; prev_w) (row vocab), then a zero row; fcur [vocab+1, d] = RMSNorm(E[v];
 * cur_w), then a zero row.  The per-row halves of TokenRouterFeatures.forward
 * (ffnmem/memory/router.py:50-59, model.RMSNorm rounding ffnmem/model.py:39-48), which depend on
 * the token id only: formed once per weight version, read by lng_router_codes_ids. */
int lng_router_feature_tables(const void* emb, int64_t vocab, int32_t d, const void* start, const void* prev_w,
                              const void* cur_w, float eps, void* fprev, void* fcur, void* stream);

/* Route codes of the token router straight from token ids: the router GEMM + sign-pack of
 * lng_router_codes over x[p] = concat(fprev[x_{t-1}] (fprev[vocab] = start at t = 0),
 * fcur[x_t], ssm_bf16[p]) with the rows gathered inside the GEMM, so the [B*T, 2d+N] features of
 * lng_router_features are never written.  Replaces TokenRouterFeatures.forward
 * (ffnmem/memory/router.py:50-59) + LngramMemory.route_logits and its quantisation
 * (ffnmem/memory/wrapper.py:98-109; lngram_v2.py:1012-1017); the codes equal those of
 * lng_router_features + lng_router_codes bit for bit.  An id outside [0, vocab) reads a zero row.
 * token_ids int64 [B*T]; ssm_bf16 [B*T, N] bf16 (lng_ssm_scan_with_bf16) or null with N = 0;
 * w [n_out, 2d+N] bf16; codes uint8 [B*T, n_out/4] (4-bit codes); logits fp32 or null.
 * Shapes: lng_router_codes_ids_ok. */
int32_t lng_router_codes_ids_ok(int64_t M, int32_t d, int32_t N, int64_t n_out);
int lng_router_codes_ids(const int64_t* token_ids, int64_t vocab, int64_t B, int64_t T, const void* fprev,
                         const void* fcur, int32_t d, const void* ssm_bf16, int32_t N, const void* w, int64_t n_out,
                         float* logits, uint8_t* codes, void* stream);

/* ---------------------------------------------------------------- K2: addresses / rows */
/* addr[B, T-order+1, R] = sum_k codes[b, t'+k, r] << (k*bits).
 * _aligned_ngram_address (lngram_v2.py:314-325).  out_dtype LNG_I32 or LNG_I64. */
int lng_ngram_address(const void* codes, int codes_dtype, int64_t B, int64_t T, int32_t R,
                      int32_t order, int32_t bits, void* out, int out_dtype, void* stream);

/* rows[B, T, route_end-route_start, n_orders] (rows_dtype LNG_I32 or LNG_I64): global
 * table row of each order-n n-gram ending at t, or -1 where _lookup_route_chunk masks it
 * to zero (lngram_v2.py:1047-1092, _valid_mask :1027-1045).  segment_ids [B,T] int32 and
 * valid_tokens [B,T] uint8 may be null.  int32 rows return LNG_E_RANGE when R * 2^(bits*n)
 * exceeds int32, where the reference's index_dtype becomes int64 (lngram_v2.py:951-959). */
int lng_ngram_rows(const void* codes, int codes_dtype, int64_t B, int64_t T, int32_t R,
                   int32_t route_start, int32_t route_end, const int32_t* orders, int32_t n_orders,
                   int32_t bits, const int32_t* segment_ids, const uint8_t* valid_tokens,
                   void* rows, int rows_dtype, void* stream);

/* Code-keyed online counts mixed into a batch of next-token distributions
 * (OnlineCounts.mix, drafting/drafters.py:117-142).  keys[T, R, n_orders]: rows of the
 * committed pairs t (row at t, token nxt[t] = x[t+1]; -1 where t < n-1); q[N, R, n_orders]:
 * the query windows' rows (-1 = invalid); pair t counts for query j iff t <= deadline[j].
 * out[N, V] = (1-lam) p + lam * sc / max(tot, 1e-9), lam = n_eff/(n_eff+kappa),
 * n_eff = tot / (R n_orders).  w_work holds N*T floats.  The count term is added with
 * atomics, so its summation order (not its value) varies between calls. */
int lng_online_mix(const int32_t* keys, const int64_t* nxt, int32_t T, const int32_t* q,
                   const int64_t* deadline, int32_t N, int32_t R, int32_t n_orders, const float* p,
                   int64_t V, float kappa, float* w_work, float* out, void* stream);

/* ---------------------------------------------------------------- K3: gather / readout */
/* Route tokens out[B, T_out, route_end-route_start, n_orders*mem_dim] in the
 * tables' dtype (LNG_F32 / LNG_BF16 / LNG_F16): _lookup_route_chunk in eval
 * (lngram_v2.py:1047-1113).  tables[i] is the [R*2^(bits*orders[i]), mem_dim]
 * table of order orders[i].  T_out = T, or target_length if > 0 (last positions). */
int lng_route_tokens(const void* codes, int codes_dtype, int64_t B, int64_t T, int32_t R,
                     int32_t route_start, int32_t route_end, const int32_t* orders, int32_t n_orders,
                     int32_t bits, const void* const* tables, int table_dtype, int32_t mem_dim,
                     const int32_t* segment_ids, const uint8_t* valid_tokens, int32_t target_length,
                     void* out, void* stream);

/* The n-gram windows of a draft tree's nodes for the memory block of tree verification
 * (tree_ngram_codes / tree_route_tokens, drafting/tree.py:114-136, as tree_verify_step uses them,
 * :179-196), with the nodes' codes cached, in one launch.  idx [n, hist+1] (int32) names each
 * window slot in cat(the last hist cached codes, the n node codes); L = L0 + *L_dev (L_dev: a
 * device int32, or null), the cached length.  Writes win [B*n, hist+1, R] u8 (the slot's code, 0
 * where the slot is a position before 0), seg [B*n, hist+1] int32 and val [B*n, hist+1] u8 (1 where
 * the slot is real: lng_route_tokens' segment ids and valid tokens for those windows), the node
 * codes [B, n, R] into cache [B, max_len, R] u8 at positions L .. L+n-1, and slots [n, n_rel] =
 * rel + L (int32; the conv windows of lng_causal_conv_slots).  The caller keeps L + n <= max_len
 * (checked here when L_dev is null). */
int lng_tree_windows(const void* node_codes, int node_codes_dtype, uint8_t* cache, int64_t B, int64_t max_len,
                     int32_t R, int32_t n, int32_t hist, const int32_t* idx, int64_t L0, const int32_t* L_dev,
                     const int32_t* rel, int32_t n_rel, uint8_t* win, int32_t* seg, uint8_t* val, int32_t* slots,
                     void* stream);

/* out[rows, dim] = RMSNorm(x) * w with one of the reference's two roundings:
 * LNG_NORM_MODEL  model.RMSNorm (model.py:39-48): normalise in fp32, round to the storage
 *                 dtype, multiply by w, round;
 * LNG_NORM_FUSED  lngram_v2.RMSNorm (lngram_v2.py:36-53, F.rms_norm): normalise and multiply
 *                 by w in fp32, round once.
 * The two agree in fp32. */
enum { LNG_NORM_MODEL = 0, LNG_NORM_FUSED = 1 };
int lng_rmsnorm(const void* x, const void* w, int dtype, int64_t rows, int32_t dim, float eps, int32_t mode,
                void* out, void* stream);

/* Decode-step projections written straight into caches (the cache writes of memory_step,
 * ffnmem/infer.py:158, :177): row m = b * group + i (i < group) of x . w^T lands at row
 * b * stride + p0 + i of the output, p0 = pos0 (+ *pos0_dev, a device int32).  bf16 operands,
 * M <= 64 (a multiple of group), N % 16 == 0, K % 32 == 0.  lng_linear_at writes bf16 rows of N
 * (the conv-input cache, from readout_o_proj); lng_router_codes_at writes the N/4 4-bit route codes
 * (uint8) of LngramMemory.route_logits + quantize_route_logits (wrapper.py:98-101,
 * lngram_v2.py:1012-1017) into the code cache.  Results equal lng_linear / lng_router_codes. */
int lng_linear_at(const void* x, const void* w, int64_t M, int64_t N, int64_t K, int64_t group, int64_t stride,
                  int64_t pos0, const int32_t* pos0_dev, void* y, void* stream);
int lng_router_codes_at(const void* x, const void* w, int64_t M, int64_t K, int64_t N, int64_t group,
                        int64_t stride, int64_t pos0, const int32_t* pos0_dev, uint8_t* codes, void* stream);

/* y[M,N] = x[M,K] . w[N,K]^T in `dtype` (fp32 accumulation, output rounded to
 * dtype).  nn.Linear without bias as used by readout_q_proj / readout_kv_proj /
 * readout_o_proj (lngram_v2.py:1115-1131, :1354-1359) and the draft head.
 * bf16 at M >= 1024, N >= 256, K >= 256 runs on hipBLASLt (host-side plan, see the
 * conventions above); M <= 64 on the skinny MFMA kernel; the rest on the tiled MFMA
 * kernels.  fp32 runs in fp32 FMA. */
int lng_linear(const void* x, const void* w, int dtype, int64_t M, int64_t N, int64_t K, void* y,
               void* stream);

/* RouteNgramMemoryV2._manual_gqa (lngram_v2.py:1899-1920) with the sink
 * denominator of _real_route_probabilities (:1887-1897): query [BT, KV*G, hd],
 * key/value [BT, KV, R, hd] -> out [BT, KV*G, hd].  Scores are rounded to the
 * storage dtype before the fp32 scale, probabilities before the value product. */
int lng_sink_attention(const void* query, const void* key, const void* value, int dtype, int64_t BT,
                       int32_t kv_heads, int32_t groups, int32_t R, int32_t head_dim, float scale,
                       float sink_logit, void* out, void* stream);

/* Same, with element strides {bt, kv_head, route} for key and value (the head
 * dim is contiguous): accepts the permuted views _project_memory returns
 * (lngram_v2.py:1120-1131) without a copy. */
int lng_sink_attention_strided(const void* query, const void* key, const void* value, int dtype, int64_t BT,
                               int32_t kv_heads, int32_t groups, int32_t R, int32_t head_dim,
                               const int64_t* key_strides, const int64_t* value_strides, float scale,
                               float sink_logit, void* out, void* stream);

/* _real_route_probabilities (lngram_v2.py:1887-1897): probs[M,R] (fp32) from
 * scores[M,R] (fp32) with a zero-value sink logit in the denominator. */
int lng_sink_probabilities(const float* scores, int64_t M, int32_t R, float sink_logit, float* probs,
                           void* stream);

/* DepthwiseCausalConv.forward (lngram_v2.py:273-286) and, with residual != 0,
 * the _finish residual (:1354-1359): out = [mixed +] SiLU(conv_dil(RMSNorm(mixed))),
 * taps conv_w[d, K] oldest->newest, zero left padding.  mixed/out [B, T, d]. */
int lng_causal_conv(const void* mixed, const void* norm_w, const void* conv_w, int dtype, int64_t B,
                    int64_t T, int32_t d, int32_t K, int32_t dilation, float eps, int residual, void* out,
                    void* stream);

/* The same convolution over a window of cached rows (the cached decode step: memory_step's
 * conv over the cache, ffnmem/infer.py:176-182; DepthwiseCausalConv.forward_incremental,
 * lngram_v2.py:288-311): rows [B, stride, d] hold `len` rows per sequence (pre-norm conv inputs,
 * positions 0 .. len-1, zero left padding before 0); the outputs of positions p0 .. p0+n-1,
 * p0 = pos0 + (*pos0_dev if pos0_dev, a device int32, e.g. the cached length), go to
 * out [B, n, d].  Each row is normalised as lng_causal_conv does, so outputs equal the whole
 * sequence's bit for bit.  Positions at or past len produce nothing (device p0 unchecked). */
int lng_causal_conv_at(const void* rows, const void* norm_w, const void* conv_w, int dtype, int64_t B, int64_t stride,
                       int64_t len, int64_t pos0, const int32_t* pos0_dev, int64_t n, int32_t d, int32_t K,
                       int32_t dilation, float eps, int residual, void* out, void* stream);

/* The same convolution with each output's window given as rows of the cache: the ancestor-window
 * conv of a draft tree's verification (drafting/tree.py:186-194, over the slots of tree_slots
 * :96-111).  slots [n, back + 1] (device int32, back = (K - 1) * dilation, oldest first): output
 * (b, i) reads tap j from row slots[i][j * dilation] of sequence b of rows [B, stride, d] and its
 * residual from row slots[i][back]; a slot outside [0, len) is a zero row (the left padding).
 * out [B, n, d].  Each shape runs the arithmetic of the kernel lng_causal_conv_at runs for it, so an
 * output equals the sequence conv's at a position whose window holds the same rows. */
int lng_causal_conv_slots(const void* rows, const void* norm_w, const void* conv_w, int dtype, int64_t B,
                          int64_t stride, int64_t len, const int32_t* slots, int64_t n, int32_t back, int32_t d,
                          int32_t K, int32_t dilation, float eps, int residual, void* out, void* stream);

/* bf16 y[M,N] = x[M,K] . w[N,K]^T (K % 32 == 0) that also writes the RMSNorm
 * statistics of its bf16 output rows for the following short conv: rowsq[p*M + m]
 * holds partial sums of squares, p < lng_linear_rowsq_partials(N).  readout_o_proj
 * feeding DepthwiseCausalConv's norm (lngram_v2.py:1354-1359, :273-286). */
int32_t lng_linear_rowsq_partials(int64_t N);
int lng_linear_rowsq(const void* x, const void* w, int64_t M, int64_t N, int64_t K, void* y, float* rowsq,
                     void* stream);

/* bf16 y[M,N] = (x[M,K] . w[N,K]^T) * rsqrt(mean_k(x[m,k]^2) + eps): a projection of RMSNorm(x),
 * the norm's weight folded into w's columns (lng_fold_columns), with each row's RMS scale formed
 * inside the GEMM from the x rows it streams.  The query projection of the fused memory readout,
 * q = W_q RMSNorm(h) (_project_query, lngram_v2.py:1115-1118), which then needs no q_rows.
 * Shapes: lng_linear_rowscale_ok(M, N, K) != 0 (M >= 1024, N >= 64, N % 8 == 0, K % 64 == 0);
 * other shapes return LNG_E_ARG. */
int32_t lng_linear_rowscale_ok(int64_t M, int64_t N, int64_t K);
int lng_linear_rowscale(const void* x, const void* w, int64_t M, int64_t N, int64_t K, float eps, void* y,
                        void* stream);

/* rowsq[m] (fp32) = sum_c x[m, c]^2 over bf16 rows [rows, d]: the RMSNorm statistic of the short
 * conv's input (DepthwiseCausalConv, lngram_v2.py:273-286) as one partial for lng_causal_conv_rowsq,
 * for output projections that do not produce it in their epilogue. */
int lng_row_sumsq(const void* x, int64_t rows, int32_t d, float* rowsq, void* stream);

/* lng_causal_conv for bf16, kernel 4, dilation 3, taking the row statistics from
 * lng_linear_rowsq instead of recomputing them (same rounding as lng_causal_conv).
 * d % 4 == 0, n_partials <= 16 (lng_linear_rowsq makes 2 per 256 output channels). */
int lng_causal_conv_rowsq(const void* mixed, const float* rowsq, int32_t n_partials, const void* norm_w,
                          const void* conv_w, int64_t B, int64_t T, int32_t d, int32_t K, int32_t dilation,
                          float eps, int residual, void* out, void* stream);

/* Fused memory readout (the metric kernel).  Replaces, in eval, the chain
 * _lookup_route_chunk -> _project_memory -> _manual_gqa of
 * RouteNgramMemoryV2.forward (lngram_v2.py:1361-1407) by the associativity
 *   score_{h,g,r} = s_r * ((w_mem . Wk[h]^T q_{h,g}) . x_r) * scale,
 *   o_{h,g}       = Wv[h] (w_mem . sum_r p_{h,g,r} s_r x_r)
 * with an online softmax seeded by the sink (m, l) = (b0, 1).  bf16 only;
 * shape: orders (2,3), mem_dim 128, 16 query heads x 64, 4 KV heads.
 *   q        [N_tok, 16*64]  projected query (readout_q_proj output)
 *   q_rows   null, or [N_tok, 16*64] bf16: the query projection's input rows, when q was projected
 *            from them with readout_query_norm.weight folded into readout_q_proj.weight
 *            (lng_fold_columns); the kernel then scales each token's query by its row's
 *            rsqrt(mean(row^2) + q_eps), which completes that RMSNorm (lngram_v2.py:1115-1118)
 *   codes    [B, T, R] uint8 route codes
 *   table2   [R*256, 128], table3 [R*4096, 128]
 *   kv_pack  [LNG_READOUT_PACK_ELEMS] bf16, readout_kv_proj.weight in the kernel's operand
 *            order, made by lng_memory_readout_pack (once per weight version)
 *   w_mem    [256]           readout_memory_norm.weight
 *   head_out [N_tok, 16*64]  attention output (input of readout_o_proj) */
#define LNG_READOUT_PACK_ELEMS 131072
int lng_memory_readout_fused(const void* q, const void* q_rows, float q_eps, const uint8_t* codes, int64_t B,
                             int64_t T, int32_t R, const void* table2, const void* table3, const void* kv_pack,
                             const void* w_mem, float eps, float scale, float sink_logit, void* head_out,
                             void* stream);

/* lng_memory_readout_fused for n new positions of B sequences after a cached prefix
 * (memory_step, ffnmem/infer.py:152-176; static_verify's memory part, live_spec.py:100-114):
 * q / q_rows / head_out [B*n, 16*64] hold the new positions; codes [B, codes_len, R] is the code
 * cache (or a verification context, infer.py:163-165) and the new tokens sit at positions
 * p0 .. p0+n-1 of it, p0 = pos0 + (*pos0_dev if pos0_dev, a device int32); their n-gram rows read
 * the codes at t, t-1, t-2 (valid from position n-1 up).  Positions outside [0, codes_len) read
 * no rows. */
int lng_memory_readout_fused_at(const void* q, const void* q_rows, float q_eps, const uint8_t* codes, int64_t B,
                                int64_t n, int32_t R, int64_t codes_len, int64_t pos0, const int32_t* pos0_dev,
                                const void* table2, const void* table3, const void* kv_pack, const void* w_mem,
                                float eps, float scale, float sink_logit, void* head_out, void* stream);

/* The fused readout over route tokens the caller supplies instead of codes and tables
 * (memory_step with route_tokens, ffnmem/infer.py:167-171: rows from host-RAM serving or staged
 * verify blocks).  route_tokens [B*n, R, 256] bf16 (the 2-gram row, then the 3-gram row; zeros
 * where the lookup masks, as _lookup_route_chunk gives them); q / q_rows / head_out as in
 * lng_memory_readout_fused.  Same arithmetic as the code path, so equal rows give equal outputs.
 * B * n * R < 2^23. */
int lng_memory_readout_fused_rows(const void* q, const void* q_rows, float q_eps, const void* route_tokens, int64_t B,
                                  int64_t n, int32_t R, const void* kv_pack, const void* w_mem, float eps, float scale,
                                  float sink_logit, void* head_out, void* stream);

/* out[N, K] = w[N, K] * s[K] (bf16, one rounding): a row RMSNorm's weight folded into the projection
 * that follows it (readout_query_norm.weight into readout_q_proj.weight, lngram_v2.py:1115-1118). */
int lng_fold_columns(const void* w, const void* s, int64_t N, int64_t K, void* out, void* stream);

/* kv_pack [LNG_READOUT_PACK_ELEMS] bf16 from readout_kv_proj.weight kv [512, 256] bf16 (rows
 * 0..255 the keys, 256..511 the values of the 4 KV heads, lngram_v2.py:1120-1131): the key
 * and value weights rearranged so that every weight load of lng_memory_readout_fused reads
 * one contiguous kilobyte.  A pure permutation (no arithmetic). */
int lng_memory_readout_pack(const void* kv, void* kv_pack, void* stream);

/* out[B*T, mem_dim] (fp32) = sum over routes r and orders n (t >= n-1) of table_n[row, :] with
 *   row = (r * S + slot) * 2^(bits n) + addr_n,   S = 2^scale_log2,
 *   addr_n = sum_k (codes[b, t-n+1+k, r] & (2^bits-1)) << (bits k)      (oldest code least significant),
 *   slot = mix32(seed ^ mix32((b*T + t) * 0x9E3779B1 + r*n_orders + i)) & (S-1)  (i = order index,
 *   mix32 = MurmurHash3 fmix32, uint32 arithmetic).
 * The row gather of _lookup_route_chunk (lngram_v2.py:1058, :1064-1092) with its zero rows for
 * t < n-1, over tables grown S times per route (the scaled-table configuration of
 * serving/scaled_tables.py:1-22 kept at R routes), summed instead of read out.  S = 1 gives the
 * reference's global rows r*16^n + addr.  tables[i] (bf16 or fp32, [R*S*2^(bits n_i), mem_dim])
 * must hold every row; mem_dim * element size must be 16 B times a divisor of 64. */
int lng_gather_sum_scaled(const void* const* tables, int table_dtype, int32_t mem_dim, const uint8_t* codes,
                          int64_t B, int64_t T, int32_t R, const int32_t* orders, int32_t n_orders, int32_t bits,
                          int32_t scale_log2, uint32_t seed, float* out, void* stream);

/* Route-logit gradient of the lookup surrogate for one n-gram order: the backward of
 * _LngramSurrogate (ffnmem/memory/lngram_v2.py:328-464; approximate mode :430-447, exact mode
 * :394-429).  grad_memory, hard_memory [B, T, R, mem_dim] in mem_dtype (f32 or bf16, the table's
 * dtype); q_logits [B, T, R, bits] (f32 or bf16); codes [B, T, R] (u8, i32 or i64) of routes
 * route_start .. route_start + R - 1; table [table_rows, mem_dim] (the order's table, rows
 * (route_start + r) * 2^(bits*order) + address); valid_mask [B, T] (the reference's _valid_mask,
 * null = all valid).  Writes grad_q [B, T, R, bits] in out_dtype (f32 or bf16): the per-bit
 * counterfactual scores times scale * temperature * p(1-p) (exact = 0), or the alphabet-wide
 * expectation derivative (exact = 1), p = sigmoid(temperature * q).  Zero when T < order,
 * temperature == 0 or scale == 0.  mem_dim in {32, 64, 128, 256}; 1 <= order <= 4, bits <= 8.
 * Each output is a fixed sum in the reference's order (no atomics).  hard_memory may be null when
 * it is the lookup's own rows (table[row] * valid[b, t], as _lookup_route_chunk makes it,
 * lngram_v2.py:1084-1090): the looked-up row of every window with a gradient is then read from
 * the table (the same bits), which saves streaming [B, T, R, mem_dim] from memory. */
int lng_surrogate_grad(const void* grad_memory, const void* hard_memory, int mem_dtype, const void* q_logits,
                       int q_dtype, const void* codes, int codes_dtype, const void* table, int64_t table_rows,
                       const uint8_t* valid_mask, int64_t B, int64_t T, int32_t R, int32_t route_start,
                       int32_t mem_dim, int32_t order, int32_t bits, float temperature, float scale, int exact,
                       void* grad_q, int out_dtype, void* stream);

/* lng_surrogate_grad with a workspace (same reference function, _LngramSurrogate.backward,
 * lngram_v2.py:364-464): for the shapes lng_surrogate_workspace_bytes gives a size for (order 3,
 * bf16 rows of 128, 4-bit codes, approximate mode, R <= 256, B*T <= 65536) the windows of every route
 * are binned by the code at their newest position, so that a block reads the looked-up and eight
 * of the twelve counterfactual rows of its windows from one 64 KB sub-block of the table held on
 * chip; the workspace holds a route-major copy of the codes and every window's twelve scores, each
 * written by the call before it is read (no clearing needed; calls that share a workspace must be
 * ordered, e.g. on one stream).  The binned path needs a 256-byte aligned workspace and 16-byte
 * aligned rows, logits and gradient (8-byte for bf16 logits and gradient); other buffers and
 * other shapes (size 0) take lng_surrogate_grad's path and ignore the workspace.  The result is a
 * fixed sum per output in
 * the reference's order, as lng_surrogate_grad's (the within-row summation order differs, so the
 * two paths agree to fp32 rounding). */
size_t lng_surrogate_workspace_bytes(int64_t B, int64_t T, int32_t R, int32_t mem_dim, int32_t order, int32_t bits,
                                     int mem_dtype, int exact);
int lng_surrogate_grad_ws(const void* grad_memory, const void* hard_memory, int mem_dtype, const void* q_logits,
                          int q_dtype, const void* codes, int codes_dtype, const void* table, int64_t table_rows,
                          const uint8_t* valid_mask, int64_t B, int64_t T, int32_t R, int32_t route_start,
                          int32_t mem_dim, int32_t order, int32_t bits, float temperature, float scale, int exact,
                          void* workspace, size_t workspace_bytes, void* grad_q, int out_dtype, void* stream);

/* Table gradient of one order's lookup: the embedding backward behind _LngramSurrogate's
 * pass-through of the memory gradient (lngram_v2.py:1084-1092, :454).  table_grad
 * [table_rows, mem_dim] fp32 (the caller zeroes it) += grad_memory[b, t, r, :] at row
 * (route_start + r) * 2^(bits*order) + address of the window ending at t, for t >= order-1 and
 * valid_mask[b, t] (null = all valid).  fp32 atomics: rows met several times sum in a varying
 * order.  mem_dim in {32, 64, 128, 256}. */
int lng_table_grad(const void* grad_memory, int mem_dtype, const void* codes, int codes_dtype,
                   const uint8_t* valid_mask, int64_t B, int64_t T, int32_t R, int32_t route_start, int32_t mem_dim,
                   int32_t order, int32_t bits, int64_t table_rows, float* table_grad, void* stream);

/* ---------------------------------------------------------------- serving layout and host-RAM rows */
/* Device address of pinned host memory (hipHostGetDevicePointer): the serving movers below read
 * host-RAM tables through it (zero-copy over the host link).  LNG_E_HIP for memory that is not
 * pinned and mapped.  No reference counterpart: the reference stages rows through host copies
 * (serving/prefetch.py:1-45, its transfer mode (ii) ZeroCopyGather is not implemented, :600-608). */
int lng_host_device_pointer(const void* host_ptr, void** dev_ptr);

/* Serving layout of one order's table (permute_table, serving/layout.py:38-43): dst row
 * (r, j) = src row (r, rev(j)), rev reversing the `order` base-2^bits digits of j.  An involution:
 * the same call maps back (restore_tables, prefetch.py:253-260).  [routes * 2^(bits*order),
 * mem_dim] in dtype (f32, bf16, f16; rows a multiple of 16 bytes); src and dst distinct. */
int lng_permute_table(const void* src, void* dst, int dtype, int32_t routes, int32_t order, int32_t bits,
                      int32_t mem_dim, void* stream);

/* out[B, T-order+1, R] int64 = sum_m codes[b, t'+order-1-m, r] << (m*bits): the address with the
 * current code least significant (serving_address, serving/layout.py:52-63). */
int lng_serving_address(const void* codes, int codes_dtype, int64_t B, int64_t T, int32_t R, int32_t order,
                        int32_t bits, int64_t* out, void* stream);

/* Exact route tokens of n new positions from serving-layout tables (LayerTable.exact_index +
 * gather, serving/prefetch.py:184-199, :226-233; serving_route_tokens, layout.py:66-81):
 * tables[k] = order orders[k]'s serving table (device or mapped host memory, table_rows[k] rows);
 * ctx [B, h + n, R] = h history codes, then the n new positions' codes, the first new position being
 * absolute position `start` (h <= start).  out [B, n, R, n_orders * mem_dim] in table_dtype,
 * zeros where the n-gram does not fit (position < order - 1). */
int lng_serving_gather(const void* const* tables, const int64_t* table_rows, int table_dtype, int32_t mem_dim,
                       const int32_t* orders, int32_t n_orders, int32_t bits, const void* ctx, int codes_dtype,
                       int64_t B, int64_t h, int64_t n, int32_t R, int64_t start, void* out, void* stream);

/* Contiguous candidate blocks of position `position` (candidate_rows / candidate_base,
 * serving/layout.py:84-108; LayerTable.candidate_index, prefetch.py:201-215): hist [B, h, R] =
 * the codes ending at position - 1.  out [B, R, n_orders, 2^bits, mem_dim]: rows base .. base + 2^bits
 * - 1 of each order's serving table; zeros where the n-gram does not fit. */
int lng_serving_candidates(const void* const* tables, const int64_t* table_rows, int table_dtype, int32_t mem_dim,
                           const int32_t* orders, int32_t n_orders, int32_t bits, const void* hist, int codes_dtype,
                           int64_t B, int64_t h, int32_t R, int64_t position, void* out, void* stream);

/* out[N, mem_dim] = table[idx[N]] (LayerTable.gather, serving/prefetch.py:226-233: one
 * index_select of a serving table, here by the device from device or mapped host memory); an
 * index outside [0, table_rows) gives a zero row. */
int lng_gather_rows(const void* table, int64_t table_rows, int dtype, int32_t mem_dim, const int64_t* idx, int64_t N,
                    void* out, void* stream);

/* out[M, R, n_orders * mem_dim] = cand[M, R, k, codes[M, R], :] (select_candidates,
 * serving/layout.py:111-116). */
int lng_select_candidates(const void* cand, int dtype, int32_t mem_dim, const void* codes, int codes_dtype,
                          int64_t M, int32_t R, int32_t n_orders, int32_t bits, void* out, void* stream);

/* ---------------------------------------------------------------- K4: SSM scan */
/* s[B,T,N] (fp32): s_t = a*s_{t-1} + (1-a)*u_t, s_{-1} = s0[B,N] (zero if null).
 * chunked_scan / sequential_scan (ffnmem/memory/ssm.py:58-91) and the carried
 * state of ssm_continue (ffnmem/infer.py:125-137), in one pass over u.  `workspace`
 * (workspace_bytes >= lng_ssm_workspace_bytes(B, T, N)) holds the tiles' hand-off
 * records; zero it once before its first use.  The kernel keeps the epoch that tags each call's
 * records in the workspace's header and advances it at the end of every call, so one workspace
 * serves any number of calls, replays of a captured HIP graph included; calls that share a
 * workspace must not overlap.  A tile whose wait for its predecessors' records runs out forms its
 * carry from u directly (exact, slow) and sets bit 0 of the int32 at byte 0 of the workspace (the
 * caller may read and clear it). */
size_t lng_ssm_workspace_bytes(int64_t B, int64_t T, int32_t N);
int lng_ssm_scan(const float* a, const float* u, const float* s0, int64_t B, int64_t T, int32_t N,
                 void* workspace, size_t workspace_bytes, float* s, void* stream);

/* lng_ssm_scan that also writes the states rounded to bf16 (s_bf16 [B, T, N]): the SSM columns
 * of the token router's features, which TokenRouterFeatures casts to the feature dtype
 * (ffnmem/memory/router.py:58), for lng_router_codes_ids. */
int lng_ssm_scan_with_bf16(const float* a, const float* u, const float* s0, int64_t B, int64_t T, int32_t N,
                           void* workspace, size_t workspace_bytes, float* s, void* s_bf16, void* stream);

/* The SSM states of a draft tree's nodes (the parent-ordered recurrence of tree_verify_step,
 * drafting/tree.py:153-161): s[b, i] = a * s[b, parent[i]] + (1 - a) * u[b, i] for the n nodes in
 * index order, with lng_ssm_scan's step, so a node's state equals the scan's along its root path.
 * parent [n] (device int32); a parent outside [0, i) -- the root's -1 -- continues from
 * s_root [B, N] (the state before the tree), or from zero when s_root is null.  u, s [B, n, N]. */
int lng_ssm_tree(const float* a, const float* u, const float* s_root, const int32_t* parent, int64_t B, int32_t n,
                 int32_t N, float* s, void* stream);

/* lng_ssm_scan with the wait for predecessor records bounded by `spin_limit` short sleeps per tile
 * (lng_ssm_scan uses a bound far past any real wait; 0 never waits, so every tile whose
 * predecessors have not yet published forms its carry from u directly).  No counterpart in the
 * reference: it lets tests drive the direct-carry path from the host. */
int lng_ssm_scan_bounded(const float* a, const float* u, const float* s0, int64_t B, int64_t T, int32_t N,
                         void* workspace, size_t workspace_bytes, int32_t spin_limit, float* s, void* stream);

/* lng_ssm_scan without a workspace argument and without any allocation: the hand-off records live
 * in a static device array of the library (8.4 MB per GPU, held until the process ends), which
 * limits the shape to B * ceil(N/256) * ceil(T/128) <= 2048 tiles (LNG_E_ARG beyond).  No
 * counterpart in the reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops).  Every call on one GPU shares that GPU's array, so calls that
 * overlap on one GPU (other streams, other threads) race; calls in one stream are fine, and so are
 * replays of a graph that captured it (its epoch lives in the array, not in the launch). */
int lng_ssm_scan_static(const float* a, const float* u, const float* s0, int64_t B, int64_t T, int32_t N,
                        float* s, void* stream);

/* The static array's status word (bit 0: a call formed some tile's carry directly, see
 * lng_ssm_scan), read after the device has finished its work and then cleared (synchronous). */
int lng_ssm_scan_static_status(int32_t* status);

/* ---------------------------------------------------------------- K5: drafting */
/* A token-routed drafter (the per-token algorithm of RefDrafter, drafting/cpu_drafter.py:76-289,
 * and of drafter.cpp:152-545) over caller-owned device buffers.  Weights are the bundle arrays
 * (export_drafter.py:22-31) plus three precomposed fp32 matrices of the draft readout:
 *   qk  [q_heads*Dt, d] = softmax_scale * diag(mem_norm) Wk[h]^T W_q[qh] diag(q_norm)
 *   qks [q_heads*Dt, N] = softmax_scale * diag(mem_norm) Wk[h]^T W_sq[qh]      (query_ssm)
 *   ov  [d, q_heads*Dt] = W_o[:, qh] Wv[h] diag(mem_norm)        (qh = h*groups + g)
 * State rows: token id, route codes [R] and SSM state [N] per position.  Rows 0 .. L-1 are
 * the committed positions, *length holds L on the device; rows past the committed capacity
 * hold hypothetical and tree positions.  A row spec names a row: v >= 0 absolute, v < 0 the
 * committed row L + v (-1 = last committed), LNG_ROW_NONE = before the sequence start. */
#define LNG_ROW_NONE (-2147483647 - 1)
#define LNG_DR_MAX_D 2048
#define LNG_DR_MAX_N 256
#define LNG_DR_MAX_DT 256
#define LNG_DR_MAX_QH 16
#define LNG_DR_MAX_CH 8
#define LNG_DR_MAX_P 16
#define LNG_DR_MAX_K 8
#define LNG_DR_SYNC_INTS 4160  /* int32 entries of lng_drafter.sync */

typedef struct lng_drafter {
  int32_t d, V, R, bits, mem_dim, dt, n_orders, orders[4], maxn;
  int32_t q_heads, kv_heads, head_dim, ssm_dim, router_ssm, query_ssm;
  int32_t emb_dtype, table_dtype, router_dtype;
  float router_eps, ssm_eps, draft_eps, mem_eps, sink_logit;
  const void* emb;                      /* [V, d]                      */
  const void* tables[4];                /* [R * 2^(bits*n), mem_dim]   */
  const void* router;                   /* [R*bits, 2d (+N)]           */
  const float* router_start;            /* [d] (fp32, like every vector below) */
  const float* router_prev_norm;
  const float* router_cur_norm;
  const float* ssm_norm;                /* [d]     (ssm_dim > 0)       */
  const float* ssm_w_in;                /* [N, d]                      */
  const float* ssm_decay;               /* [N]                         */
  const float* qk;
  const float* qks;
  const float* ov;
  const float* out_norm;                /* [d]                         */
  int64_t* tokens;                      /* [rows]                      */
  uint8_t* codes;                       /* [rows, R]                   */
  float* ssm;                           /* [rows, N]                   */
  const int32_t* length;                /* device int32: L             */
  int32_t rows;
  /* Per-token tables of the token-only drafter (router_ssm == query_ssm == 0).  When every one
   * is non-null the readout runs in two launches per call:
   *   lut_prev  [V, R*bits] fp32   router[:, :d]   (RMSNorm(E[v]) * prev_norm)
   *   lut_cur   [V, R*bits] fp32   router[:, d:2d] (RMSNorm(E[v]) * cur_norm)
   *   lut_start [R*bits]    fp32   router[:, :d]   (RMSNorm(start) * prev_norm)
   *   lut_qk    [V, q_heads*Dt] fp32   qk (E[v] * rsqrt(mean(E[v]^2) + draft_eps))
   *   lut_out   [V, q_heads*hd] fp32   E[v] diag(out_norm) W_o
   *   gram_out  [q_heads*hd, q_heads*hd] fp32   W_o^T W_o
   *   wv_t      [kv_heads, Dt, hd] (wv_dtype)   Wv[h]^T, the value rows of kv_proj transposed
   *   mem_norm  [Dt] fp32   readout_memory_norm weight
   *   sync      int32 [LNG_DR_SYNC_INTS], zero before the first call; every call leaves it
   *             zero (block counters, online totals and per-block candidate counts).  Any
   *             drafter may set it: readouts of at most 4 positions then run the small-batch
   *             kernels (one weight row per wave, route chunks merged by the last block). */
  const float* lut_prev;
  const float* lut_cur;
  const float* lut_start;
  const float* lut_qk;
  const float* lut_out;
  const float* gram_out;
  const void* wv_t;
  const float* mem_norm;
  int32_t wv_dtype;
  int32_t* sync;
  /* Optional (may be null): lut_out in the vocabulary kernel's MFMA operand order, fp32
   * [ceil(V/16)][q_heads*hd/16][64][4]: element (t, s, l, e) = lut_out[16t + l%16][16s + 4(l/16) + e]
   * (zero past row V-1), so that each load of a 16-row tile moves one contiguous kilobyte. */
  const float* lut_out_pk;
} lng_drafter;

/* sizeof(lng_drafter), for bindings that mirror the struct. */
size_t lng_drafter_size(void);

/* Bytes of `work` for up to `max_positions` (<= LNG_DR_MAX_P) readout positions, top-k <=
 * `max_k`, online counts over up to `max_pairs` committed pairs. */
size_t lng_drafter_workspace_bytes(const lng_drafter* D, int32_t max_positions, int32_t max_k, int32_t max_pairs);

/* Process n new positions: SSM step and router codes (cpu_drafter.py:147-164,
 * drafter.cpp:396-425).  List form: rows[j] / prev[j] are row specs (prev = the previous
 * position, LNG_ROW_NONE for the first token of a sequence), n <= LNG_DR_MAX_P; positions are
 * processed in order, so a position may follow an earlier one of the same call.  Range form:
 * absolute rows base .. base+n-1 in sequence, the first after prev0.  With
 * codes_from_router == 0 the codes rows are left as written by the caller (commit with the
 * target's codes). */
int lng_drafter_advance(const lng_drafter* D, const int32_t* rows, const int32_t* prev, int32_t n,
                        int codes_from_router, void* work, size_t work_bytes, void* stream);
int lng_drafter_advance_range(const lng_drafter* D, int32_t base, int32_t prev0, int32_t n, int codes_from_router,
                              void* work, size_t work_bytes, void* stream);

/* Draft readout + full-vocabulary top-k for P positions (cpu_drafter.py:208-270,
 * drafter.cpp:477-556).  windows [P, maxn] (host) are row specs of each position's n-gram
 * window, oldest first, the position itself last.  ids/scores [P, k] (device) receive the
 * top-k by (logit desc, id asc); with online != 0 the logits are mixed with code-keyed online
 * counts over the committed pairs (drafters.py:117-142) and ranked by, and reported as, the
 * log of the mixed probability.  Child j of the call (child_rows/child_parent/child_rank, host,
 * n_children <= 64) receives token ids[parent][rank] (top-1 if absent) in D->tokens.
 * logits [P, V] (device) may be null.  `counts` [P, V] int32 (device) must be zero before the
 * first call; every call leaves it zero. */
int lng_drafter_readout(const lng_drafter* D, const int32_t* windows, int32_t P, int32_t k, int online, float kappa,
                        const int32_t* child_rows, const int32_t* child_parent, const int32_t* child_rank,
                        int32_t n_children, void* work, size_t work_bytes, int32_t* counts, int64_t* ids,
                        float* scores, float* logits, void* stream);

/* Route tokens [P, R, Dt] (table dtype) of the n-grams ending at each window's last position
 * (tree_route_tokens, drafting/tree.py:130-136; window_route_tokens, drafters.py:110-114). */
int lng_drafter_gather(const lng_drafter* D, const int32_t* windows, int32_t P, void* out, void* stream);

/* Count sketches of the drafter's orders (drafting/sketches.py:1-12, bundle arrays sketch_ids_<n>,
 * sketch_counts_<n>, fallback; export_drafter.py:33-34), on the device. */
typedef struct lng_sketch {
  const int32_t* ids[4];      /* per order index i (orders[i]): [R * 2^(bits*n), k] token ids, or null */
  const int64_t* counts[4];   /* same shape: counts, 0 = empty slot (null with ids)                    */
  int32_t k;                  /* slots per row                                                         */
  int32_t cap;                /* shortlist length, 1 .. 256                                            */
  const int32_t* fallback;    /* [n_fallback] padding tokens in order                                  */
  int32_t n_fallback;         /* 0 .. 1024                                                             */
} lng_sketch;

/* Sketch-shortlist drafts (RefDrafter._shortlist + _readout + draft's top-k, cpu_drafter.py:179-206,
 * :238-262; drafter.cpp:438-474) of P positions given their full-vocabulary logits [P, V] and
 * full-vocabulary top-k (ids / scores [P, k], from lng_drafter_readout with the same k): the
 * candidates are the tokens of the positions' sketch rows with counts summed per token, ordered
 * by (total desc, id asc) and cut to cap, padded with fallback tokens not yet present (ids outside
 * [0, V) are skipped); ids/scores [P, k] are their top-k logits, ties in candidate order; an empty
 * list keeps the full-vocabulary top-k.  shortlist [P, cap] int32 / shortlist_logits [P, cap]
 * (optional) receive the list (-1 / -inf pad; an empty list gives tokens 0 .. cap-1, as
 * RefDrafter.trace).  Children as lng_drafter_readout.  Needs n_orders * R * k <= 8192, R <= 256. */
int lng_drafter_shortlist(const lng_drafter* D, const lng_sketch* S, const int32_t* windows, int32_t P,
                          const float* logits, const int64_t* full_ids, const float* full_scores, int32_t k,
                          const int32_t* child_rows, const int32_t* child_parent, const int32_t* child_rank,
                          int32_t n_children, int64_t* ids, float* scores, int32_t* shortlist,
                          float* shortlist_logits, void* stream);

/* The readout and the sketch shortlist of P positions in one call (RefDrafter.draft's per-token
 * step with a shortlist: _readout of the shortlist tokens only, cpu_drafter.py:238-262;
 * drafter.cpp:438-474): the candidates are scored from the readout's hidden state, and only a
 * position whose list is empty scores the whole vocabulary.  Results as lng_drafter_readout
 * followed by lng_drafter_shortlist (same list, ids, scores and children; logits within fp32
 * rounding).  work: lng_drafter_workspace_bytes(D, P, k, .) bytes.  No online counts. */
int lng_drafter_readout_shortlist(const lng_drafter* D, const lng_sketch* S, const int32_t* windows, int32_t P,
                                  int32_t k, const int32_t* child_rows, const int32_t* child_parent,
                                  const int32_t* child_rank, int32_t n_children, void* work, size_t work_bytes,
                                  int64_t* ids, float* scores, int32_t* shortlist, float* shortlist_logits,
                                  void* stream);

/* One draft-tree step (draft_tree, drafting/tree.py:243-257, batched by depth): node 0 is the
 * last committed token, node i >= 1 lives at absolute row node_row0 + i; parent/rank (host, n
 * <= 64) as TreeSpec (tree.py:37-51).  Every parent's readout of one depth runs together;
 * node i receives the rank[i]-th candidate of its parent (top-1 if absent).  Then every node
 * gets its codes and, if route_tokens is non-null, the verification gather [n, R, Dt]
 * (tree_ngram_codes + tree_route_tokens, tree.py:114-136).  The root's token is copied to row
 * node_row0, so rows node_row0 .. node_row0+n-1 hold every node's token (tree_accept input). */
int lng_drafter_tree(const lng_drafter* D, const int32_t* parent, const int32_t* rank, int32_t n, int32_t node_row0,
                     int online, float kappa, void* work, size_t work_bytes, int32_t* counts, void* route_tokens,
                     void* stream);

/* lng_drafter_tree with the sketch shortlist choosing every child (draft_tree over a RefDrafter
 * whose draft() scores the shortlist, tree.py:243-257 with cpu_drafter.py:238-262); no online
 * counts.  logits_work: device fp32 [16, V] scratch. */
int lng_drafter_tree_shortlist(const lng_drafter* D, const lng_sketch* S, const int32_t* parent, const int32_t* rank,
                               int32_t n, int32_t node_row0, void* work, size_t work_bytes, float* logits_work,
                               void* route_tokens, void* stream);

/* Draft tree with verification gather in one launch for the whole tree (drafting/tree.py:243-257 draft_tree
 * over cpu_drafter.py:208-270 readouts and drafters.py:117-142 online counts; tree.py:96-136
 * tree_route_tokens), for token-only drafters with the per-token tables at the SD drafters' shape:
 * q_heads 4, head_dim 64, orders (2, 3) with mem_dim 128, bits 4, R <= 192, bf16 tables and value
 * weight, V <= 32832; trees of at most 32 nodes, 8 depths, 4 parents per depth and rank < 4.
 * Same outputs as lng_drafter_tree (node tokens and codes in rows node_row0 + i, the root token in
 * row node_row0, route_tokens [n, R, 256] bf16 when not null).  One grid of resident blocks runs
 * every depth: at depth d the attention blocks select their node's token from depth d-1's
 * vocabulary records, gather its window and attend per query head; vocabulary blocks hold their
 * lut_out slice in registers for the whole tree, count the online matches of the pairs whose next
 * token they own, and score the slice once the depth's attention records arrive through
 * device-coherent (value, tag) pairs; leaf blocks gather the leaves' verification rows.  Every wait
 * is bounded.  `work` holds lng_drafter_tree_levels_workspace(D) bytes, zero before the first call
 * and kept between calls (its first word holds the call epoch; the int32 at byte offset 4 is an
 * error word: non-zero = a wait timed out, and the call's outputs are then not to be used: read it
 * after the call, and on non-zero zero the workspace and redo the call with lng_drafter_tree; a
 * non-zero int32 at byte offset 8 asks for per-block phase times of the 100 MHz clock in the
 * workspace's last section).  The workspace size is 0, and the call returns LNG_E_ARG without
 * launching, for a drafter or tree outside the limits above (lng_drafter_tree runs those). */
size_t lng_drafter_tree_levels_workspace(const lng_drafter* D);
int lng_drafter_tree_levels(const lng_drafter* D, const int32_t* parent, const int32_t* rank, int32_t n,
                            int32_t node_row0, int online, float kappa, void* work, size_t work_bytes,
                            void* route_tokens, void* stream);


/* Tree acceptance (drafting/tree.py:205-220): from the root take the first child
 * (index order) whose token equals argmax[cur]; repeat.  path[n] receives the
 * node path (root first), *path_len its length, new_tokens[n] the accepted
 * tokens followed by argmax at the last path node (path_len entries). */
int lng_tree_accept(const int32_t* parent, const int64_t* node_tokens, const int64_t* argmax, int32_t n,
                    int32_t* path, int32_t* path_len, int64_t* new_tokens, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LNGRAM_HIP_H */
