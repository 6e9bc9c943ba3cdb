// CPU drafter port -- TEST INFRASTRUCTURE ONLY (the oracle's C++ restatement of the reference's
// C++ drafter, drafting/cpu/drafter.cpp, and the CPU baseline bench.py times beside the GPU
// drafter).  Nothing in the product links it.
//
// Per token it follows drafter.cpp:396-545 (the same algorithm as RefDrafter,
// drafting/cpu_drafter.py:147-289):
//   advance : SSM step s = a s + (1-a) W_in RMSNorm(E[x])            (drafter.cpp:400-406)
//             router logits W_r concat(RMSNorm(E[x_prev] | start), RMSNorm(E[x])[, s]),
//             code bit i of route r = logit[r*bits + i] > 0            (:407-421)
//   rows    : r * 2^(bits n) + sum_k code[t-n+1+k] << (bits k)         (:427-436)
//   readout : per route RMSNorm(rows) -> kv_proj; query W_q RMSNorm(E[x]) (+ W_sq s); sink
//             softmax over routes per query head; W_o; RMSNorm; logits E . h  (:477-545)
//   top-k   : (logit desc, id asc)                                    (:547-556)
// fp32 arithmetic (RMSNorm sums of squares in double, like drafter.cpp:113-118), tables bf16
// or fp32 (the reference takes fp16/fp32; bf16 is the table type of the configurations timed
// here).  Routes and vocabulary rows are split over OpenMP threads; every output element is
// computed by one thread with the same arithmetic, so results do not depend on the thread count.
//
// Optional code-keyed online counts (drafting/drafters.py:117-142): the draft softmax is mixed
// with next-token counts of the committed (row at t, token t+1) pairs whose row equals the query's
// row, per (order, route); candidates are ranked by the mixed probability, reported as its log.
//
// C API (cdr_*): the caller keeps every weight array alive for the drafter's lifetime (the
// reference's drafter keeps references to its tensors the same way, drafter.cpp:558).
#include <omp.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <mutex>
#include <string>
#include <vector>

extern "C" {

typedef struct {
  int32_t d, V, R, bits, mem_dim, kv_heads, head_dim, q_heads, ssm_dim, n_orders, orders[4];
  int32_t router_ssm, query_ssm, table_bf16;
  float router_eps, ssm_eps, draft_eps, mem_eps, softmax_scale, sink_logit;
} cdr_config;

typedef struct {
  const float *embedding, *mem_norm, *kv_proj, *router, *router_prev_norm, *router_cur_norm, *router_start;
  const float *ssm_norm, *ssm_w_in, *ssm_decay, *q_norm, *w_q, *w_sq, *w_o, *out_norm;
  const void* tables[4];
} cdr_weights;

}  // extern "C"

namespace {

thread_local std::string g_err;

int err(const std::string& m) {
  g_err = m;
  return -1;
}

inline float bf16_to_f32(uint16_t h) {
  uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// 8 partial sums (vectorises to one 8-wide FMA chain per accumulator)
inline float dotf(const float* a, const float* b, int64_t n) {
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int k = 0; k < 8; ++k) s[k] += a[i + k] * b[i + k];
  for (; i < n; ++i) s[0] += a[i] * b[i];
  return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

inline void matvec(const float* W, const float* x, float* y, int64_t rows, int64_t cols) {
  for (int64_t i = 0; i < rows; ++i) y[i] = dotf(W + i * cols, x, cols);
}

inline void rms(const float* x, const float* w, float eps, float* out, int64_t n) {
  double ss = 0.0;
  for (int64_t i = 0; i < n; ++i) ss += static_cast<double>(x[i]) * x[i];
  const float r = 1.0f / std::sqrt(static_cast<float>(ss / static_cast<double>(n)) + eps);
  for (int64_t i = 0; i < n; ++i) out[i] = x[i] * r * w[i];
}

struct Cursor {
  int64_t t = -1, tok = -1;
  std::vector<float> s;
  std::vector<uint8_t> hist;  // maxn x R codes, oldest first
};

class CpuDrafter {
 public:
  CpuDrafter(const cdr_config& c, const cdr_weights& w, int threads, int online, float kappa)
      : c_(c), w_(w), threads_(std::max(1, threads)), online_(online != 0), kappa_(kappa) {
    maxn_ = 0;
    for (int i = 0; i < c.n_orders; ++i) maxn_ = std::max(maxn_, c.orders[i]);
    G_ = c.q_heads / c.kv_heads;
    KH_ = c.kv_heads * c.head_dim;
    I_ = c.q_heads * c.head_dim;
    Dt_ = c.n_orders * c.mem_dim;
    N_ = c.ssm_dim;
    F_ = 2 * c.d + (c.router_ssm ? N_ : 0);
    rt_.resize(static_cast<size_t>(c.R) * Dt_);
    kv_.resize(static_cast<size_t>(c.R) * 2 * KH_);
    lg_.resize(c.V);
  }

  std::mutex mu;
  std::vector<int64_t> tokens;
  std::vector<uint8_t> codes;  // [n, R]
  std::vector<float> ssm;      // [n, N]

  int64_t length() const { return static_cast<int64_t>(tokens.size()); }
  void set_threads(int t) { threads_ = std::max(1, t); }

  int commit(const int64_t* toks, int64_t n, const uint8_t* over) {
    Cursor cur = cursor();
    for (int64_t i = 0; i < n; ++i) {
      if (toks[i] < 0 || toks[i] >= c_.V) return err("token id out of range");
      advance(cur, toks[i], over ? over + i * c_.R : nullptr);
      tokens.push_back(toks[i]);
      codes.insert(codes.end(), cur.hist.end() - c_.R, cur.hist.end());
      if (N_) ssm.insert(ssm.end(), cur.s.begin(), cur.s.end());
    }
    return 0;
  }

  // gamma greedy drafts after the committed tokens + hyp; ids/scores [gamma, k] (-1 / -inf pad),
  // codes [nh + advanced, R]; returns the number of code rows written through *n_codes.
  int draft(int gamma, const int64_t* hyp, int nh, int k, int last_codes, int64_t* toks, int64_t* ids,
            float* scores, uint8_t* out_codes, int* n_codes) {
    Cursor cur = cursor();
    if (cur.t < 0 && nh == 0) return err("draft needs at least one committed or hypothetical token");
    const int64_t n_pairs = std::max<int64_t>(length() - 1, 0);
    int ci = 0;
    for (int i = 0; i < nh; ++i) {
      if (hyp[i] < 0 || hyp[i] >= c_.V) return err("token id out of range");
      advance(cur, hyp[i], nullptr);
      std::copy(cur.hist.end() - c_.R, cur.hist.end(), out_codes + static_cast<int64_t>(ci++) * c_.R);
    }
    std::vector<int64_t> top;
    for (int i = 0; i < gamma; ++i) {
      distribution(cur, n_pairs);
      top_order(k, top);
      for (int j = 0; j < k; ++j) {
        const bool ok = j < static_cast<int>(top.size());
        ids[i * k + j] = ok ? top[j] : -1;
        scores[i * k + j] = ok ? lg_[top[j]] : -std::numeric_limits<float>::infinity();
      }
      toks[i] = top[0];
      if (i + 1 < gamma || last_codes) {
        advance(cur, top[0], nullptr);
        std::copy(cur.hist.end() - c_.R, cur.hist.end(), out_codes + static_cast<int64_t>(ci++) * c_.R);
      }
    }
    *n_codes = ci;
    return 0;
  }

  // Teacher-forced pass from an empty state over the full vocabulary (drafter.cpp:315-370).
  int trace(const int64_t* toks, int64_t T, const uint8_t* over, uint8_t* out_codes, float* out_scores) {
    std::vector<int64_t> st;
    std::vector<uint8_t> sc;
    std::vector<float> ss;
    std::swap(st, tokens);
    std::swap(sc, codes);
    std::swap(ss, ssm);
    int rc = 0;
    Cursor cur = cursor();
    for (int64_t t = 0; t < T && rc == 0; ++t) {
      if (toks[t] < 0 || toks[t] >= c_.V) {
        rc = err("token id out of range");
        break;
      }
      advance(cur, toks[t], over ? over + t * c_.R : nullptr);
      tokens.push_back(toks[t]);
      codes.insert(codes.end(), cur.hist.end() - c_.R, cur.hist.end());
      if (N_) ssm.insert(ssm.end(), cur.s.begin(), cur.s.end());
      std::copy(cur.hist.end() - c_.R, cur.hist.end(), out_codes + t * c_.R);
      distribution(cur, t);
      std::copy(lg_.begin(), lg_.end(), out_scores + t * c_.V);
    }
    std::swap(st, tokens);
    std::swap(sc, codes);
    std::swap(ss, ssm);
    return rc;
  }

  // draft_tree (drafting/tree.py:243-257): node i = the rank[i]-th candidate after its parent's
  // path (-1 falls back to the top-1); one draft of one token per distinct parent.
  int draft_tree(const int32_t* parent, const int32_t* rank, int n, int64_t* node_tokens) {
    if (length() == 0) return err("draft_tree needs a committed token");
    int k = 1;
    for (int i = 1; i < n; ++i) {
      if (parent[i] < 0 || parent[i] >= i) return err("parent[i] must precede i");
      k = std::max(k, rank[i] + 1);
    }
    node_tokens[0] = tokens.back();
    std::vector<std::vector<int64_t>> cache(n);
    std::vector<int64_t> hyp, t1(1), ids(k);
    std::vector<float> sc(k);
    std::vector<uint8_t> cod(static_cast<size_t>(n + 1) * c_.R);
    for (int i = 1; i < n; ++i) {
      const int p = parent[i];
      if (cache[p].empty()) {
        hyp.clear();
        for (int a = p; a > 0; a = parent[a]) hyp.push_back(node_tokens[a]);
        std::reverse(hyp.begin(), hyp.end());
        int nc = 0;
        if (int rc = draft(1, hyp.data(), static_cast<int>(hyp.size()), k, 0, t1.data(), ids.data(), sc.data(),
                           cod.data(), &nc))
          return rc;
        cache[p] = ids;
      }
      const int64_t t = cache[p][rank[i]];
      node_tokens[i] = t >= 0 ? t : cache[p][0];
    }
    return 0;
  }

 private:
  Cursor cursor() const {
    Cursor c;
    c.hist.assign(static_cast<size_t>(maxn_) * c_.R, 0);
    if (N_) c.s.assign(N_, 0.f);
    const int64_t n = length();
    if (n == 0) return c;
    c.t = n - 1;
    c.tok = tokens.back();
    if (N_) std::copy(ssm.end() - N_, ssm.end(), c.s.begin());
    const int64_t h = std::min<int64_t>(n, maxn_);
    std::copy(codes.end() - h * c_.R, codes.end(), c.hist.end() - h * c_.R);
    return c;
  }

  void advance(Cursor& c, int64_t tok, const uint8_t* over) {
    const int64_t d = c_.d;
    const float* e = w_.embedding + tok * d;
    if (N_) {
      std::vector<float> xn(d), u(N_);
      rms(e, w_.ssm_norm, c_.ssm_eps, xn.data(), d);
      matvec(w_.ssm_w_in, xn.data(), u.data(), N_, d);
      for (int i = 0; i < N_; ++i) c.s[i] = w_.ssm_decay[i] * c.s[i] + (1.f - w_.ssm_decay[i]) * u[i];
    }
    std::vector<uint8_t> code(c_.R, 0);
    if (over) {
      std::copy(over, over + c_.R, code.begin());
    } else {
      std::vector<float> feat(F_), lg(static_cast<size_t>(c_.R) * c_.bits);
      rms(c.t >= 0 ? w_.embedding + c.tok * d : w_.router_start, w_.router_prev_norm, c_.router_eps, feat.data(), d);
      rms(e, w_.router_cur_norm, c_.router_eps, feat.data() + d, d);
      if (c_.router_ssm) std::copy(c.s.begin(), c.s.end(), feat.begin() + 2 * d);
      matvec(w_.router, feat.data(), lg.data(), static_cast<int64_t>(c_.R) * c_.bits, F_);
      for (int r = 0; r < c_.R; ++r) {
        int v = 0;
        for (int b = 0; b < c_.bits; ++b) v |= (lg[r * c_.bits + b] > 0.f ? 1 : 0) << b;
        code[r] = static_cast<uint8_t>(v);
      }
    }
    std::copy(c.hist.begin() + c_.R, c.hist.end(), c.hist.begin());
    std::copy(code.begin(), code.end(), c.hist.end() - c_.R);
    c.t += 1;
    c.tok = tok;
  }

  // row of route r, order index oi of the n-gram ending at the cursor (-1 before t = n-1)
  int64_t row(const Cursor& c, int oi, int r) const {
    const int n = c_.orders[oi];
    if (c.t < n - 1) return -1;
    int64_t addr = 0;
    for (int k = 0; k < n; ++k) addr |= static_cast<int64_t>(c.hist[static_cast<size_t>(maxn_ - n + k) * c_.R + r]) << (k * c_.bits);
    return static_cast<int64_t>(r) * (int64_t{1} << (c_.bits * n)) + addr;
  }

  // key row of the committed n-gram ending at position t (-1 before t = n-1)
  int64_t key(int64_t t, int oi, int r) const {
    const int n = c_.orders[oi];
    if (t < n - 1) return -1;
    int64_t addr = 0;
    for (int k = 0; k < n; ++k) addr |= static_cast<int64_t>(codes[static_cast<size_t>(t - n + 1 + k) * c_.R + r]) << (k * c_.bits);
    return static_cast<int64_t>(r) * (int64_t{1} << (c_.bits * n)) + addr;
  }

  // lg_ = draft logits at the cursor (or the log of the online-mixed probability)
  void distribution(const Cursor& c, int64_t n_pairs) {
    const int R = c_.R, md = c_.mem_dim, no = c_.n_orders;
    const int64_t d = c_.d, V = c_.V;
    std::vector<int64_t> rows(static_cast<size_t>(no) * R);
    for (int oi = 0; oi < no; ++oi)
      for (int r = 0; r < R; ++r) rows[static_cast<size_t>(oi) * R + r] = row(c, oi, r);
    // 1. route tokens -> memory norm -> KV (routes over threads)
#pragma omp parallel for num_threads(threads_) schedule(static)
    for (int r = 0; r < R; ++r) {
      float* tok = rt_.data() + static_cast<size_t>(r) * Dt_;
      for (int oi = 0; oi < no; ++oi) {
        float* dst = tok + oi * md;
        const int64_t rw = rows[static_cast<size_t>(oi) * R + r];
        if (rw < 0) {
          std::fill(dst, dst + md, 0.f);
        } else if (c_.table_bf16) {
          const uint16_t* src = static_cast<const uint16_t*>(w_.tables[oi]) + rw * md;
          for (int j = 0; j < md; ++j) dst[j] = bf16_to_f32(src[j]);
        } else {
          const float* src = static_cast<const float*>(w_.tables[oi]) + rw * md;
          std::copy(src, src + md, dst);
        }
      }
      rms(tok, w_.mem_norm, c_.mem_eps, tok, Dt_);
      matvec(w_.kv_proj, tok, kv_.data() + static_cast<size_t>(r) * 2 * KH_, 2 * KH_, Dt_);
    }
    // 2. query
    const float* e = w_.embedding + c.tok * d;
    std::vector<float> xn(d), q(I_), out(I_, 0.f), sc(R), hid(d), hn(d);
    rms(e, w_.q_norm, c_.draft_eps, xn.data(), d);
    matvec(w_.w_q, xn.data(), q.data(), I_, d);
    if (c_.query_ssm && w_.w_sq) {
      std::vector<float> tmp(I_);
      matvec(w_.w_sq, c.s.data(), tmp.data(), I_, N_);
      for (int i = 0; i < I_; ++i) q[i] += tmp[i];
    }
    // 3. sink softmax over routes per query head (qh = h * G + g)
    const int hd = c_.head_dim;
    for (int h = 0; h < c_.kv_heads; ++h)
      for (int g = 0; g < G_; ++g) {
        const float* qv = q.data() + (h * G_ + g) * hd;
        float mx = c_.sink_logit;
        for (int r = 0; r < R; ++r) {
          sc[r] = dotf(qv, kv_.data() + static_cast<size_t>(r) * 2 * KH_ + h * hd, hd) * c_.softmax_scale;
          mx = std::max(mx, sc[r]);
        }
        float den = 0.f;
        for (int r = 0; r < R; ++r) {
          sc[r] = std::exp(sc[r] - mx);
          den += sc[r];
        }
        den += std::exp(c_.sink_logit - mx);
        float* o = out.data() + (h * G_ + g) * hd;
        for (int r = 0; r < R; ++r) {
          const float p = sc[r] / den;
          const float* v = kv_.data() + static_cast<size_t>(r) * 2 * KH_ + KH_ + h * hd;
          for (int j = 0; j < hd; ++j) o[j] += p * v[j];
        }
      }
    // 4. output projection + norm, 5. full-vocabulary logits (rows over threads)
    matvec(w_.w_o, out.data(), hid.data(), d, I_);
    rms(hid.data(), w_.out_norm, c_.draft_eps, hn.data(), d);
#pragma omp parallel for num_threads(threads_) schedule(static)
    for (int64_t v = 0; v < V; ++v) lg_[v] = dotf(w_.embedding + v * d, hn.data(), d);
    if (online_) mix_online(c, n_pairs);
  }

  // drafters.py:117-142 for one query: w[t] = sum over orders and routes of [key_n(t, r) == q_n(r)],
  // p = (1 - lam) softmax(lg) + lam sc / sum(w), lam = n_eff / (n_eff + kappa), n_eff = sum(w) / (R n).
  void mix_online(const Cursor& c, int64_t n_pairs) {
    const int R = c_.R, no = c_.n_orders;
    const int64_t V = c_.V;
    if (n_pairs <= 0) {
      // (1 - 0) softmax: the ranking of the logits, reported as log-probabilities
      softmax_log(0.0, nullptr, 0.0);
      return;
    }
    std::vector<int64_t> q(static_cast<size_t>(no) * R);
    for (int oi = 0; oi < no; ++oi)
      for (int r = 0; r < R; ++r) q[static_cast<size_t>(oi) * R + r] = row(c, oi, r);
    std::vector<int32_t> w(n_pairs, 0);
#pragma omp parallel for num_threads(threads_) schedule(static)
    for (int64_t t = 0; t < n_pairs; ++t) {
      int32_t s = 0;
      for (int oi = 0; oi < no; ++oi)
        for (int r = 0; r < R; ++r) {
          const int64_t qq = q[static_cast<size_t>(oi) * R + r];
          s += (qq >= 0 && key(t, oi, r) == qq) ? 1 : 0;
        }
      w[t] = s;
    }
    std::vector<double> cnt(V, 0.0);
    double tot = 0.0;
    for (int64_t t = 0; t < n_pairs; ++t) {
      cnt[tokens[t + 1]] += w[t];
      tot += w[t];
    }
    const double n_eff = tot / (static_cast<double>(R) * no);
    const double lam = n_eff / (n_eff + kappa_);
    softmax_log(lam, cnt.data(), std::max(tot, 1e-9));
  }

  void softmax_log(double lam, const double* cnt, double tot) {
    const int64_t V = c_.V;
    float m = -std::numeric_limits<float>::infinity();
    for (int64_t v = 0; v < V; ++v) m = std::max(m, lg_[v]);
    double s = 0.0;
    for (int64_t v = 0; v < V; ++v) s += std::exp(static_cast<double>(lg_[v] - m));
    for (int64_t v = 0; v < V; ++v) {
      double p = (1.0 - lam) * std::exp(static_cast<double>(lg_[v] - m)) / s;
      if (cnt) p += lam * cnt[v] / tot;
      lg_[v] = static_cast<float>(std::log(p));
    }
  }

  void top_order(int k, std::vector<int64_t>& idx) const {
    const int64_t V = c_.V;
    idx.resize(V);
    for (int64_t i = 0; i < V; ++i) idx[i] = i;
    const int64_t m = std::min<int64_t>(k, V);
    std::partial_sort(idx.begin(), idx.begin() + m, idx.end(),
                      [&](int64_t a, int64_t b) { return lg_[a] != lg_[b] ? lg_[a] > lg_[b] : a < b; });
    idx.resize(m);
  }

  cdr_config c_;
  cdr_weights w_;
  int threads_;
  bool online_;
  float kappa_;
  int maxn_, G_, KH_, I_, Dt_, N_, F_;
  std::vector<float> rt_, kv_, lg_;
};

}  // namespace

extern "C" {

const char* cdr_last_error(void) { return g_err.c_str(); }

void* cdr_create(const cdr_config* c, const cdr_weights* w, int threads, int online, float kappa) {
  if (!c || !w || c->n_orders < 1 || c->n_orders > 4 || c->q_heads % c->kv_heads || c->bits < 1 || c->bits > 8) {
    err("cdr_create: bad config");
    return nullptr;
  }
  return new CpuDrafter(*c, *w, threads, online, kappa);
}

void cdr_destroy(void* h) { delete static_cast<CpuDrafter*>(h); }

int64_t cdr_length(void* h) { return static_cast<CpuDrafter*>(h)->length(); }

void cdr_set_threads(void* h, int threads) {
  auto* d = static_cast<CpuDrafter*>(h);
  std::lock_guard<std::mutex> g(d->mu);
  d->set_threads(threads);
}

void cdr_reset(void* h) {
  auto* d = static_cast<CpuDrafter*>(h);
  std::lock_guard<std::mutex> g(d->mu);
  d->tokens.clear();
  d->codes.clear();
  d->ssm.clear();
}

int cdr_truncate(void* h, int64_t n, int32_t R, int32_t N) {
  auto* d = static_cast<CpuDrafter*>(h);
  std::lock_guard<std::mutex> g(d->mu);
  if (n < 0 || n > d->length()) return err("cannot truncate beyond the committed length");
  d->tokens.resize(n);
  d->codes.resize(static_cast<size_t>(n) * R);
  d->ssm.resize(static_cast<size_t>(n) * N);
  return 0;
}

int cdr_commit(void* h, const int64_t* toks, int64_t n, const uint8_t* codes) {
  auto* d = static_cast<CpuDrafter*>(h);
  std::lock_guard<std::mutex> g(d->mu);
  return d->commit(toks, n, codes);
}

int cdr_draft(void* h, int gamma, const int64_t* hyp, int nh, int k, int last_codes, int64_t* toks, int64_t* ids,
              float* scores, uint8_t* codes, int* n_codes) {
  auto* d = static_cast<CpuDrafter*>(h);
  std::lock_guard<std::mutex> g(d->mu);
  return d->draft(gamma, hyp, nh, k, last_codes, toks, ids, scores, codes, n_codes);
}

int cdr_trace(void* h, const int64_t* toks, int64_t T, const uint8_t* codes, uint8_t* out_codes, float* out_scores) {
  auto* d = static_cast<CpuDrafter*>(h);
  std::lock_guard<std::mutex> g(d->mu);
  return d->trace(toks, T, codes, out_codes, out_scores);
}

int cdr_draft_tree(void* h, const int32_t* parent, const int32_t* rank, int n, int64_t* node_tokens) {
  auto* d = static_cast<CpuDrafter*>(h);
  std::lock_guard<std::mutex> g(d->mu);
  return d->draft_tree(parent, rank, n, node_tokens);
}

}  // extern "C"
