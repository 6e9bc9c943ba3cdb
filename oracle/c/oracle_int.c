/*
 * oracle_int.c -- C restatement of the integer parts of the route n-gram memory
 * hot path.  TEST INFRASTRUCTURE ONLY: the checker the HIP kernels and the Python
 * oracle are compared against; never linked into the product.
 *
 * Functions (reference file:line each restates):
 *   orc_pack_codes     lngram_v2.py:74-89 + :1012-1017 (sign bits -> route codes)
 *   orc_ngram_rows     lngram_v2.py:314-325, :1027-1045, :1047-1092 (rows, -1 = zero row)
 *   orc_tree_slots     drafting/tree.py:96-111 (ancestor windows)
 *   orc_tree_accept    drafting/tree.py:205-220 (greedy tree acceptance)
 *   orc_online_weights drafting/drafters.py:129-142 (code-keyed online count weights)
 */
#include <stdint.h>
#include <string.h>

void orc_pack_codes(const float* logits, int64_t M, int32_t routes, int32_t bits, int32_t* codes) {
  for (int64_t m = 0; m < M; ++m)
    for (int32_t r = 0; r < routes; ++r) {
      int32_t v = 0;
      for (int32_t i = 0; i < bits; ++i)
        if (logits[(m * routes + r) * bits + i] > 0.0f) v |= 1 << i;
      codes[m * routes + r] = v;
    }
}

/* rows[B,T,R,n_orders]; seg [B,T] or NULL; valid [B,T] or NULL */
void orc_ngram_rows(const int32_t* codes, int64_t B, int64_t T, int32_t R, const int32_t* orders,
                    int32_t n_orders, int32_t bits, const int32_t* seg, const uint8_t* valid, int64_t* rows) {
  for (int64_t b = 0; b < B; ++b)
    for (int64_t t = 0; t < T; ++t)
      for (int32_t r = 0; r < R; ++r)
        for (int32_t oi = 0; oi < n_orders; ++oi) {
          const int32_t n = orders[oi];
          int64_t row = -1;
          if (t >= n - 1) {
            const int64_t t0 = t - n + 1;
            int ok = 1;
            if (seg && seg[b * T + t0] != seg[b * T + t]) ok = 0;
            if (valid && !valid[b * T + t]) ok = 0;
            if (ok) {
              int64_t addr = 0;
              for (int32_t k = 0; k < n; ++k) addr |= (int64_t)codes[(b * T + t0 + k) * R + r] << (k * bits);
              row = (int64_t)r * ((int64_t)1 << (bits * n)) + addr;
            }
          }
          rows[((b * T + t) * R + r) * n_orders + oi] = row;
        }
}

/* idx/ok [n, back+1]: slot of each node's j-th predecessor along its ancestors (oldest first),
 * continuing into the L positions before the root; slot L + a = node a. */
void orc_tree_slots(const int32_t* parent, int32_t n, int64_t L, int32_t back, int64_t* idx, uint8_t* ok) {
  int32_t path[256];
  for (int32_t i = 0; i < n; ++i) {
    int32_t len = 0, a = i;
    while (a >= 0 && len < 256) {
      path[len++] = a;
      a = parent[a];
    } /* path[0] = i, path[len-1] = root */
    for (int32_t j = 0; j <= back; ++j) {
      int64_t s;
      if (j < len)
        s = L + path[j];
      else
        s = L - (j - len + 1);
      const int32_t col = back - j;
      idx[i * (back + 1) + col] = s >= 0 ? s : 0;
      ok[i * (back + 1) + col] = s >= 0;
    }
  }
}

/* Returns path length; path[len], new_tokens[len]. */
int32_t orc_tree_accept(const int32_t* parent, int32_t n, const int64_t* node_tokens, const int64_t* argmax,
                        int32_t* path, int64_t* new_tokens) {
  int32_t cur = 0, len = 1;
  path[0] = 0;
  for (;;) {
    int32_t nxt = -1;
    for (int32_t c = 0; c < n; ++c)
      if (parent[c] == cur && node_tokens[c] == argmax[cur]) {
        nxt = c;
        break;
      }
    if (nxt < 0) break;
    path[len++] = nxt;
    cur = nxt;
  }
  for (int32_t i = 1; i < len; ++i) new_tokens[i - 1] = node_tokens[path[i]];
  new_tokens[len - 1] = argmax[cur];
  return len;
}

/* w[j, t] = sum_{n, r} [keys_n[t, r] == q_n[j, r] && q_n[j, r] >= 0] * [t <= deadline[j]]
 * keys [n_orders, P, R] (pairs t = 0..P-1), q [n_orders, J, R], w [J, P] (float). */
void orc_online_weights(const int64_t* keys, const int64_t* q, int32_t n_orders, int64_t P, int64_t J, int32_t R,
                        const int64_t* deadline, float* w) {
  memset(w, 0, sizeof(float) * (size_t)(J * P));
  for (int64_t j = 0; j < J; ++j)
    for (int64_t t = 0; t < P; ++t) {
      if (t > deadline[j]) continue;
      int64_t cnt = 0;
      for (int32_t o = 0; o < n_orders; ++o)
        for (int32_t r = 0; r < R; ++r) {
          const int64_t qq = q[(o * J + j) * R + r];
          if (qq >= 0 && keys[(o * P + t) * R + r] == qq) ++cnt;
        }
      w[j * P + t] = (float)cnt;
    }
}
