/*
 * WKV7 fp64 CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker for the HIP product path. Only tests/, the smoke()
 * entry of __graft_entry__.py and the cpu_baseline leg of bench.py may load
 * it. The product path (flashrwkv_amd) never links, loads or calls it.
 *
 * It restates, in plain fp64 loops, the naive recurrence the reference uses as
 * its own parity target:
 *   /root/reference/tests/tmix/wkv7/test.py:157-213      (fp32-state oracle)
 *   /root/reference/tests/tmix/wkv7/statetune/test.py:39-88 (boundary and
 *       state_dot_a definitions: boundary = state at each chunk start,
 *       state_dot_a[t] = a_t^T S_{t-1})
 * and the adjoint recurrence whose per-token gradient definitions are those
 * of /root/reference/csrc/sm90/tmix/wkv7/statetune_recurrent_fp32io16_backward.cu:139-242,
 * except that S_{t-1} comes from the stored forward states (never from
 * dividing by the decay).
 *
 * State layout is [K,V]: state[k][v], as the reference pool
 * (csrc/sm120/tmix/wkv7/infer_recurrent_fp32io16_forward_varlen.cu:132-140).
 * Per token, with w the retention (already transformed from logits):
 *   sa[v]   = sum_k a[k] S[k][v]
 *   S[k][v] = w[k] S[k][v] + b[k] sa[v] + k[k] v[v]
 *   y[v]    = scale * sum_k r[k] S[k][v]
 *
 * Work is organised as sequences made of segments (token ranges). Inference
 * varlen calls pass one segment per sequence; StateTune passes its chunk
 * metadata. Every (sequence, head) pair is independent, so they may be spread
 * over OpenMP threads without changing any result.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* exp(-exp(-1/2) * sigmoid(x)): recurrent_decay.cuh:18-22, test.py:173,200. */
double wkv7o_retention_from_logits(double x) {
  const double sig = 1.0 / (1.0 + exp(-x));
  return exp(-exp(-0.5) * sig);
}

/* d log(retention) / dx = -exp(-1/2) sigmoid (1 - sigmoid): recurrent_decay.cuh:27-32. */
double wkv7o_retention_log_derivative(double x) {
  const double sig = 1.0 / (1.0 + exp(-x));
  return -exp(-0.5) * sig * (1.0 - sig);
}

void wkv7o_retention_from_logits_array(const double* x, const double* bias,
                                       int64_t rows, int64_t width,
                                       double* out) {
  for (int64_t i = 0; i < rows; ++i) {
    for (int64_t j = 0; j < width; ++j) {
      double value = x[i * width + j];
      if (bias) value += bias[j];
      out[i * width + j] = wkv7o_retention_from_logits(value);
    }
  }
}

static int64_t tok(int64_t t, int h, int H, int D) {
  return ((int64_t)t * H + h) * D;
}

/* One token step on state s (D x D, [K,V]). Writes sa and y. */
static void step(int D, double* s, const double* r, const double* w,
                 const double* k, const double* v, const double* a,
                 const double* b, double scale, double* sa, double* y) {
  for (int j = 0; j < D; ++j) {
    double acc = 0.0;
    for (int i = 0; i < D; ++i) acc += a[i] * s[i * D + j];
    sa[j] = acc;
  }
  for (int i = 0; i < D; ++i) {
    for (int j = 0; j < D; ++j) {
      s[i * D + j] = w[i] * s[i * D + j] + b[i] * sa[j] + k[i] * v[j];
    }
  }
  for (int j = 0; j < D; ++j) {
    double acc = 0.0;
    for (int i = 0; i < D; ++i) acc += r[i] * s[i * D + j];
    y[j] = scale * acc;
  }
}

/*
 * Forward. state is indexed by state_slots[seq] (slot pool, [*,H,D,D]) and
 * updated in place. boundary (optional) receives the state at the start of
 * every segment, indexed by global segment number. state_dot_a (optional)
 * receives sa per token.
 */
void wkv7o_forward(int32_t num_sequences, int32_t num_heads, int32_t head_size,
                   const int32_t* seg_offsets, const int32_t* seg_starts,
                   const int32_t* seg_ends, const int32_t* state_slots,
                   double* state, const double* r, const double* w,
                   const double* k, const double* v, const double* a,
                   const double* b, double scale, double* y, double* boundary,
                   double* state_dot_a, int num_threads) {
  const int H = num_heads, D = head_size;
  const int64_t units = (int64_t)num_sequences * H;
#ifdef _OPENMP
  if (num_threads > 0) omp_set_num_threads(num_threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
  for (int64_t u = 0; u < units; ++u) {
    const int seq = (int)(u / H), h = (int)(u % H);
    double* s = state + ((int64_t)state_slots[seq] * H + h) * D * D;
    double sa[256], yy[256];
    for (int32_t seg = seg_offsets[seq]; seg < seg_offsets[seq + 1]; ++seg) {
      if (boundary) {
        memcpy(boundary + ((int64_t)seg * H + h) * D * D, s,
               sizeof(double) * D * D);
      }
      for (int32_t t = seg_starts[seg]; t < seg_ends[seg]; ++t) {
        const int64_t o = tok(t, h, H, D);
        step(D, s, r + o, w + o, k + o, v + o, a + o, b + o, scale, sa, yy);
        memcpy(y + o, yy, sizeof(double) * D);
        if (state_dot_a) memcpy(state_dot_a + o, sa, sizeof(double) * D);
      }
    }
  }
  (void)num_threads;
}

/*
 * Backward of wkv7o_forward for loss L(y, S_final). initial_state holds S0
 * per slot (not modified). dy and dstate_final may be NULL (zero). Outputs
 * dL/dr, dL/dw (w = retention), dL/dk, dL/dv, dL/da, dL/db per token and
 * dL/dS0 per slot (dstate0, same indexing as initial_state).
 */
void wkv7o_backward(int32_t num_sequences, int32_t num_heads, int32_t head_size,
                    const int32_t* seg_offsets, const int32_t* seg_starts,
                    const int32_t* seg_ends, const int32_t* state_slots,
                    const double* initial_state, const double* r,
                    const double* w, const double* k, const double* v,
                    const double* a, const double* b, double scale,
                    const double* dy, const double* dstate_final, double* dr,
                    double* dw, double* dk, double* dv, double* da, double* db,
                    double* dstate0, int num_threads) {
  const int H = num_heads, D = head_size;
  const int64_t units = (int64_t)num_sequences * H;
#ifdef _OPENMP
  if (num_threads > 0) omp_set_num_threads(num_threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
  for (int64_t u = 0; u < units; ++u) {
    const int seq = (int)(u / H), h = (int)(u % H);
    const int64_t sbase = ((int64_t)state_slots[seq] * H + h) * D * D;
    /* Token list of this sequence, in forward order. */
    int64_t ntok = 0;
    for (int32_t seg = seg_offsets[seq]; seg < seg_offsets[seq + 1]; ++seg) {
      if (seg_ends[seg] > seg_starts[seg]) ntok += seg_ends[seg] - seg_starts[seg];
    }
    int32_t* toks = (int32_t*)malloc(sizeof(int32_t) * (ntok > 0 ? ntok : 1));
    int64_t n = 0;
    for (int32_t seg = seg_offsets[seq]; seg < seg_offsets[seq + 1]; ++seg) {
      for (int32_t t = seg_starts[seg]; t < seg_ends[seg]; ++t) toks[n++] = t;
    }
    /* states[i] = S after i tokens of this sequence (states[0] = S0). */
    double* states = (double*)malloc(sizeof(double) * D * D * (ntok + 1));
    memcpy(states, initial_state + sbase, sizeof(double) * D * D);
    double sa[256], yy[256], dsa[256];
    for (int64_t i = 0; i < ntok; ++i) {
      double* s = states + (i + 1) * D * D;
      memcpy(s, states + i * D * D, sizeof(double) * D * D);
      const int64_t o = tok(toks[i], h, H, D);
      step(D, s, r + o, w + o, k + o, v + o, a + o, b + o, scale, sa, yy);
    }
    double* adj = (double*)malloc(sizeof(double) * D * D);
    if (dstate_final) {
      memcpy(adj, dstate_final + sbase, sizeof(double) * D * D);
    } else {
      memset(adj, 0, sizeof(double) * D * D);
    }
    for (int64_t i = ntok - 1; i >= 0; --i) {
      const int64_t o = tok(toks[i], h, H, D);
      const double* s_new = states + (i + 1) * D * D;
      const double* s_old = states + i * D * D;
      const double *rt = r + o, *wt = w + o, *kt = k + o, *vt = v + o,
                   *at = a + o, *bt = b + o;
      /* y_t = scale S_t^T r_t contributes scale r_t dy_t^T to dL/dS_t. */
      if (dy) {
        const double* g = dy + o;
        for (int i2 = 0; i2 < D; ++i2)
          for (int j = 0; j < D; ++j) adj[i2 * D + j] += scale * rt[i2] * g[j];
        for (int i2 = 0; i2 < D; ++i2) {
          double acc = 0.0;
          for (int j = 0; j < D; ++j) acc += s_new[i2 * D + j] * g[j];
          dr[o + i2] = scale * acc;
        }
      } else {
        for (int i2 = 0; i2 < D; ++i2) dr[o + i2] = 0.0;
      }
      for (int j = 0; j < D; ++j) {
        double acc = 0.0;
        for (int i2 = 0; i2 < D; ++i2) acc += at[i2] * s_old[i2 * D + j];
        sa[j] = acc;
      }
      for (int j = 0; j < D; ++j) {
        double acc_v = 0.0, acc_sa = 0.0;
        for (int i2 = 0; i2 < D; ++i2) {
          acc_v += adj[i2 * D + j] * kt[i2];
          acc_sa += adj[i2 * D + j] * bt[i2];
        }
        dv[o + j] = acc_v;
        dsa[j] = acc_sa;
      }
      for (int i2 = 0; i2 < D; ++i2) {
        double acc_k = 0.0, acc_b = 0.0, acc_w = 0.0, acc_a = 0.0;
        for (int j = 0; j < D; ++j) {
          const double A = adj[i2 * D + j];
          acc_k += A * vt[j];
          acc_b += A * sa[j];
          acc_w += A * s_old[i2 * D + j];
          acc_a += s_old[i2 * D + j] * dsa[j];
        }
        dk[o + i2] = acc_k;
        db[o + i2] = acc_b;
        dw[o + i2] = acc_w;
        da[o + i2] = acc_a;
      }
      /* dL/dS_{t-1} = diag(w) A + a dsa^T */
      for (int i2 = 0; i2 < D; ++i2)
        for (int j = 0; j < D; ++j)
          adj[i2 * D + j] = wt[i2] * adj[i2 * D + j] + at[i2] * dsa[j];
    }
    memcpy(dstate0 + sbase, adj, sizeof(double) * D * D);
    free(adj);
    free(states);
    free(toks);
  }
  (void)num_threads;
}

/* Number of OpenMP threads available (1 without OpenMP). */
int wkv7o_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
