/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle of the sparse projection -> activation -> pool path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and
 * only as the checker.  The product path (granulelayer_amd) never links or calls it.
 *
 * It restates the reference's Mode-A arithmetic (every neuron owns its own fan-in record) in plain
 * C with float64 accumulation, so fp32 GPU results are compared against a more exact value:
 *
 *   z[b,n]  = sum_k x[b, idx[n,k]] * w[n,k] + bias[n]
 *             sparse_pooling/reference/pytorch_reference.py:29-47 (Mode-A branch :43-46),
 *             sparse_pooling/kernels/triton_fused.py:253-264 (_tile_z Mode A)
 *   a       = act(z)                 pytorch_reference.py:19-26 (identity | relu | exact GELU)
 *   pre[b,g]= scale_g * sum_{s < n_g} a[b, g*S+s]
 *             mean: scale_g = 1/n_g   pytorch_reference.py:78-79, kernels/ops.py:198-199
 *             sum : scale_g = 1       (mean * n_g; BASELINE's "sum pooling")
 *   backward (kernels/ops.py:242-249 dense_coefficients, triton_fused.py:364-374 _dz_from_z,
 *             triton_fused.py:402-445 _bwd_tile Mode A, autograd.py:399-414):
 *     c1[b,g] = dy[b,g] * scale_g ;  dz[b,n] = c1 * act'(z)   (relu: z > 0, so 0 at z == 0)
 *     db[n]  += sum_b dz ;  dW[n,k] += sum_b dz * x[b, idx[n,k]] ;  dX[b, idx[n,k]] += dz * w[n,k]
 *   padded slots (s >= n_g) are masked out of every sum (triton_fused.py:330-338, 428-431).
 *
 *   max pooling (pool 2; pytorch_reference.py:61-67, merge_finalize kernels/ops.py:189-195,
 *   triton_fused.py:129-139 _update max):
 *     pre[b,g] = max_{s < n_g} a[b, g*S+s];  winner[b,g] = the smallest slot s attaining it
 *     backward (autograd of the gather, the event backward autograd.py:284-289): only the winner
 *     gets a gradient:  dz[b, winner] = dy[b,g] * act'(z[b, winner])
 *
 *   top-k mean pooling (pool 3; pytorch_reference.py:68-77): the slots of the k largest raw z
 *   (stable descending sort: ties to the smaller slot), kk = min(n_g, k);
 *     pre[b,g] = sum of act(z) over the first kk of them / kk
 *     backward (autograd.py:290-295): dz = dy[b,g] / kk * act'(z) for the kk selected neurons
 *
 *   smooth pooling (pools 4 LogMeanExp, 5 power mean, 6 softmax-weighted; pytorch_reference.py:80-100):
 *     LME (temperature tau):  pre = tau * (logsumexp(a / tau) - log n_g)
 *     power (p >= 1, a = relu(z) >= 0): pre = M * (mean_n (a_n / M)^p)^(1/p), M = max a (0 if M == 0)
 *     softmax-weighted (beta): pre = sum_n softmax(beta a)_n * a_n
 *     the base-2 log-normaliser L2 = log2 sum_n 2^(u_n), u = a * scale, scale = log2(e) / tau (LME),
 *     log2(e) * beta (softmax-weighted) (kernels/ops.py:74-79, 201-209)
 *     backward (kernels/ops.py:242-262 dense_coefficients, triton_fused.py:364-399 _dz_from_z):
 *       LME:     dz = dy * 2^(u - L2) * act'(z)
 *       power:   dz = pre > 0 ? dy / n_g * (a / pre)^(p - 1) : 0, for z > 0
 *       softmax: dz = dy * 2^(u - L2) * (1 + beta (a - pre)) * act'(z)
 *
 *   Adam (sparse_pooling/optim.py:26-64, fp32 parameters: HAS_MASTER=False, STOCH=False):
 *     m = b1*m + (1-b1)*g ; v = b2*v + (1-b2)*g*g ; upd = (m/bc1) / (sqrt(v/bc2) + eps)
 *     p = p*(1 - lr*wd) - lr*upd ; g = 0        evaluated in fp32, in this order, unfused.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off), output oracle/_build/libgl_oracle.so.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* act 0 identity, 1 relu, 2 exact (erf) GELU: 0.5 z (1 + erf(z / sqrt 2)), derivative
 * Phi(z) + z phi(z) (triton_fused.py:29-45 _act / _dact, pytorch_reference.py:19-26 F.gelu) */
static inline double act_f(double z, int act) {
  if (act == 2) return 0.5 * z * (1.0 + erf(z * 0.70710678118654752440));
  return act == 1 ? (z > 0.0 ? z : 0.0) : z;
}
static inline double dact_f(double z, int act) {
  if (act == 2) return 0.5 * (1.0 + erf(z * 0.70710678118654752440)) + z * 0.39894228040143267794 * exp(-0.5 * z * z);
  return act == 1 ? (z > 0.0 ? 1.0 : 0.0) : 1.0;
}

/* Pre-activation of neuron n for token row xb (float64 accumulation in k order); *mag receives
 * sum_k |x w| + |bias|, the scale of the fp32 rounding error of z. */
static inline double neuron_z(const float* xb, const int32_t* idx, const float* w, const float* bias, long n, int K,
                              double* mag) {
  double z = 0.0, m = 0.0;
  for (int k = 0; k < K; ++k) {
    double t = (double)xb[idx[n * K + k]] * (double)w[n * K + k];
    z += t;
    m += fabs(t);
  }
  if (mag) *mag = m + fabs((double)bias[n]);
  return z + (double)bias[n];
}

/*
 * Forward.  x [B, D] fp32 (bf16 inputs are widened exactly by the caller); idx/w [G*S, K];
 * bias [G*S]; counts [G]; pool 0 = mean, 1 = sum (max: glo_forward_max_f64); act 0 = identity, 1 = relu,
 * 2 = GELU.
 * pre [B, G] float64.  mag (optional, [B, G]): scale_g * sum_s (sum_k |x w| + |bias|), the
 * magnitude the rounding error of an fp32 evaluation of pre is proportional to.
 */
void glo_forward_f64(int B, int D, int G, int S, int K, const float* x, const int32_t* idx, const float* w,
                     const float* bias, const int32_t* counts, int act, int pool, double* pre, double* mag) {
  for (int b = 0; b < B; ++b) {
    const float* xb = x + (size_t)b * D;
    for (int g = 0; g < G; ++g) {
      double s = 0.0, m = 0.0, zm;
      int n_g = counts[g];
      for (int sl = 0; sl < n_g; ++sl) {
        s += act_f(neuron_z(xb, idx, w, bias, (long)g * S + sl, K, &zm), act);
        m += zm;
      }
      pre[(size_t)b * G + g] = pool == 0 ? s / (double)n_g : s;
      if (mag) mag[(size_t)b * G + g] = pool == 0 ? m / (double)n_g : m;
    }
  }
}

/*
 * Max pooling forward (pool 2).  pre [B, G] float64, winner [B, G] int32 (pool-local slot), and
 * gap [B, G] (optional): (best - second best) / (scale of the fp32 rounding of z), the margin by
 * which an fp32 evaluation of the two leading values could swap them (+inf for a single neuron).
 * Ties go to the smaller slot, as torch.argmax returns the first maximum.
 */
void glo_forward_max_f64(int B, int D, int G, int S, int K, const float* x, const int32_t* idx, const float* w,
                         const float* bias, const int32_t* counts, int act, double* pre, int32_t* winner,
                         double* gap) {
  for (int b = 0; b < B; ++b) {
    const float* xb = x + (size_t)b * D;
    for (int g = 0; g < G; ++g) {
      const int n_g = counts[g];
      double best = -INFINITY, second = -INFINITY, mag = 0.0;
      int win = 0;
      for (int sl = 0; sl < n_g; ++sl) {
        double zm;
        const double a = act_f(neuron_z(xb, idx, w, bias, (long)g * S + sl, K, &zm), act);
        if (zm > mag) mag = zm;
        if (a > best) {
          second = best;
          best = a;
          win = sl;
        } else if (a > second) {
          second = a;
        }
      }
      pre[(size_t)b * G + g] = best;
      winner[(size_t)b * G + g] = win;
      if (gap) gap[(size_t)b * G + g] = n_g < 2 ? INFINITY : (best - second) / (mag > 0.0 ? mag : 1.0);
    }
  }
}

/* slots of the kk = min(n_g, k) largest z of pool g for token row xb, best first (ties: smaller
 * slot); returns kk.  z[s] for s < n_g must hold the pool's pre-activations. */
static int topk_select(const double* z, int n_g, int k, int* sel) {
  const int kk = n_g < k ? n_g : k;
  for (int j = 0; j < kk; ++j) {
    int best = -1;
    for (int s = 0; s < n_g; ++s) {
      int taken = 0;
      for (int i = 0; i < j; ++i) taken |= sel[i] == s;
      if (taken) continue;
      if (best < 0 || z[s] > z[best]) best = s;  /* strict: the first (smaller) slot keeps ties */
    }
    sel[j] = best;
  }
  return kk;
}

/*
 * Top-k mean pooling forward (pool 3).  pre [B, G] float64; slots [B, G, k] int32 (the selected
 * pool slots, best first, -1 past kk = min(n_g, k)); gap [B, G] (optional): (z of the kk-th
 * selected - the best unselected z) / (scale of the fp32 rounding of z), the margin by which an
 * fp32 evaluation could change the selected set (+inf when every neuron is selected).
 */
void glo_forward_topk_f64(int B, int D, int G, int S, int K, const float* x, const int32_t* idx, const float* w,
                          const float* bias, const int32_t* counts, int act, int k, double* pre, int32_t* slots,
                          double* gap) {
  double* z = (double*)malloc(sizeof(double) * (size_t)S);
  int* sel = (int*)malloc(sizeof(int) * (size_t)(k > 0 ? k : 1));
  for (int b = 0; b < B; ++b) {
    const float* xb = x + (size_t)b * D;
    for (int g = 0; g < G; ++g) {
      const int n_g = counts[g];
      double mag = 0.0;
      for (int sl = 0; sl < n_g; ++sl) {
        double zm;
        z[sl] = neuron_z(xb, idx, w, bias, (long)g * S + sl, K, &zm);
        if (zm > mag) mag = zm;
      }
      const int kk = topk_select(z, n_g, k, sel);
      double sum = 0.0, rest = -INFINITY;
      for (int j = 0; j < kk; ++j) sum += act_f(z[sel[j]], act);
      for (int sl = 0; sl < n_g; ++sl) {
        int taken = 0;
        for (int j = 0; j < kk; ++j) taken |= sel[j] == sl;
        if (!taken && z[sl] > rest) rest = z[sl];
      }
      pre[(size_t)b * G + g] = sum / (double)kk;
      for (int j = 0; j < k; ++j) slots[((size_t)b * G + g) * k + j] = j < kk ? sel[j] : -1;
      if (gap) gap[(size_t)b * G + g] = kk == n_g ? INFINITY : (z[sel[kk - 1]] - rest) / (mag > 0.0 ? mag : 1.0);
    }
  }
  free(z);
  free(sel);
}

/*
 * Backward.  dy [B, G] fp32 is dL/dpre (the out-activation of mean/sum is identity).
 * dW [G*S, K], db [G*S], dX [B, D] are float64 and ACCUMULATED (+=), like main_grad.
 *
 * Optional error-scale outputs (same shapes, accumulated; pass NULL to skip):
 *   mag*  sum of |terms| of every gradient sum (the scale of fp32 summation error);
 *   unc*  contribution of (token, neuron) pairs whose relu mask an fp32 evaluation of z may
 *         decide differently: |z| <= amb * (sum_k |x w| + |bias|).  Their terms use the float64
 *         mask in dW/db/dX and are added as |term| to unc*.
 */
static void backward_impl(int B, int D, int G, int S, int K, const float* x, const int32_t* idx, const float* w,
                          const float* bias, const int32_t* counts, int act, int pool, int topk, const float* dy,
                          double* dW, double* db, double* dX, double amb, double* magW, double* magb, double* magX,
                          double* uncW, double* uncb, double* uncX) {
  double* zb = pool == 3 ? (double*)malloc(sizeof(double) * (size_t)S) : NULL;
  int* sel = pool == 3 ? (int*)malloc(sizeof(int) * (size_t)topk) : NULL;
  for (int b = 0; b < B; ++b) {
    const float* xb = x + (size_t)b * D;
    double* dxb = dX + (size_t)b * D;
    for (int g = 0; g < G; ++g) {
      int n_g = counts[g];
      double c1 = (double)dy[(size_t)b * G + g] * (pool == 0 ? 1.0 / (double)n_g : 1.0);  /* pool 3: below */
      int win = -1;  /* max pooling: the winner (first maximum of act(z)) is the only neuron with a gradient */
      if (pool == 2) {
        double best = -INFINITY;
        for (int sl = 0; sl < n_g; ++sl) {
          const double a = act_f(neuron_z(xb, idx, w, bias, (long)g * S + sl, K, NULL), act);
          if (a > best) best = a, win = sl;
        }
      }
      int kk = 0;  /* top-k mean: the kk selected neurons, each with dy / kk */
      if (pool == 3) {
        for (int sl = 0; sl < n_g; ++sl) zb[sl] = neuron_z(xb, idx, w, bias, (long)g * S + sl, K, NULL);
        kk = topk_select(zb, n_g, topk, sel);
        c1 = (double)dy[(size_t)b * G + g] / (double)kk;
      }
      for (int sl = 0; sl < n_g; ++sl) {
        if (pool == 2 && sl != win) continue;
        if (pool == 3) {
          int taken = 0;
          for (int j = 0; j < kk; ++j) taken |= sel[j] == sl;
          if (!taken) continue;
        }
        long n = (long)g * S + sl;
        double zm;
        double z = neuron_z(xb, idx, w, bias, n, K, &zm);
        double dz = c1 * dact_f(z, act);
        int ambiguous = act == 1 && fabs(z) <= amb * zm;
        db[n] += dz;
        if (magb) magb[n] += fabs(dz);
        if (ambiguous && uncb) uncb[n] += fabs(c1);
        for (int k = 0; k < K; ++k) {
          int d = idx[n * K + k];
          dW[n * K + k] += dz * (double)xb[d];
          dxb[d] += dz * (double)w[n * K + k];
          if (magW) magW[n * K + k] += fabs(dz * (double)xb[d]);
          if (magX) magX[(size_t)b * D + d] += fabs(dz * (double)w[n * K + k]);
          if (ambiguous && uncW) uncW[n * K + k] += fabs(c1 * (double)xb[d]);
          if (ambiguous && uncX) uncX[(size_t)b * D + d] += fabs(c1 * (double)w[n * K + k]);
        }
      }
    }
  }
  free(zb);
  free(sel);
}

void glo_backward_f64(int B, int D, int G, int S, int K, const float* x, const int32_t* idx, const float* w,
                      const float* bias, const int32_t* counts, int act, int pool, const float* dy, double* dW,
                      double* db, double* dX, double amb, double* magW, double* magb, double* magX, double* uncW,
                      double* uncb, double* uncX) {
  backward_impl(B, D, G, S, K, x, idx, w, bias, counts, act, pool, 0, dy, dW, db, dX, amb, magW, magb, magX, uncW,
                uncb, uncX);
}

/*
 * Backward of a given selection (max: kpe = 1, coef = dy; top-k mean: kpe = k, coef = dy / kk with
 * kk = min(n_g, k)): slots [B, G, kpe] (-1 = none).  dz = coef * act'(z) for every listed slot,
 * accumulated into dW, db, dX (float64) with the mag* error scales.  Equal to the max / top-k
 * backward when slots is that pooling's own selection.
 */
void glo_backward_events_f64(int B, int D, int G, int S, int K, const float* x, const int32_t* idx, const float* w,
                             const float* bias, const int32_t* counts, int act, int topk_mode, int kpe,
                             const int32_t* slots, const float* dy, double* dW, double* db, double* dX, double* magW,
                             double* magb, double* magX) {
  for (int b = 0; b < B; ++b) {
    const float* xb = x + (size_t)b * D;
    for (int g = 0; g < G; ++g) {
      const int n_g = counts[g];
      const int kk = n_g < kpe ? n_g : kpe;
      const double coef = (double)dy[(size_t)b * G + g] / (topk_mode ? (double)kk : 1.0);
      for (int j = 0; j < kpe; ++j) {
        const int sl = slots[((size_t)b * G + g) * kpe + j];
        if (sl < 0 || sl >= n_g) continue;
        const long n = (long)g * S + sl;
        const double dz = coef * dact_f(neuron_z(xb, idx, w, bias, n, K, NULL), act);
        db[n] += dz;
        if (magb) magb[n] += fabs(dz);
        for (int k = 0; k < K; ++k) {
          const int d = idx[n * K + k];
          dW[n * K + k] += dz * (double)xb[d];
          dX[(size_t)b * D + d] += dz * (double)w[n * K + k];
          if (magW) magW[n * K + k] += fabs(dz * (double)xb[d]);
          if (magX) magX[(size_t)b * D + d] += fabs(dz * (double)w[n * K + k]);
        }
      }
    }
  }
}

/* top-k mean backward (pool 3) with k selected per (token, pool) */
void glo_backward_topk_f64(int B, int D, int G, int S, int K, const float* x, const int32_t* idx, const float* w,
                           const float* bias, const int32_t* counts, int act, int k, const float* dy, double* dW,
                           double* db, double* dX, double amb, double* magW, double* magb, double* magX,
                           double* uncW, double* uncb, double* uncX) {
  backward_impl(B, D, G, S, K, x, idx, w, bias, counts, act, 3, k, dy, dW, db, dX, amb, magW, magb, magX, uncW, uncb,
                uncX);
}

/* round-to-nearest-even fp32 -> bf16 -> fp32 (torch's .to(torch.bfloat16) for finite values) */
static inline float bf16_round(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) { /* inf / nan: keep, quiet nan */
    if (u & 0x007fffffu) u |= 0x00400000u;
    u &= 0xffff0000u;
  } else {
    uint32_t lsb = (u >> 16) & 1u;
    u = (u + 0x7fffu + lsb) & 0xffff0000u;
  }
  float r;
  memcpy(&r, &u, 4);
  return r;
}

/*
 * Fused AdamW step over n fp32 parameters, in place; g is zeroed (fused zero_grad).
 * moments_bf16: m, v are stored rounded to bf16 (values kept in fp32 arrays here).
 */
void glo_adam_f32(long n, float* p, float* g, float* m, float* v, float lr, float b1, float b2, float eps, float wd,
                  float bc1, float bc2, int moments_bf16) {
  for (long i = 0; i < n; ++i) {
    float gi = g[i];
    float mi = b1 * m[i] + (1.0f - b1) * gi;
    float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
    float upd = (mi / bc1) / (sqrtf(vi / bc2) + eps);
    float pi = p[i] * (1.0f - lr * wd) - lr * upd;
    m[i] = moments_bf16 ? bf16_round(mi) : mi;
    v[i] = moments_bf16 ? bf16_round(vi) : vi;
    g[i] = 0.0f;
    p[i] = pi;
  }
}

/* Philox-4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
 * SC'11; the Random123 generator): 10 rounds of (hi, lo) = M * c with the round multipliers
 * 0xD2511F53 / 0xCD9E8D57 and the Weyl key increments 0x9E3779B9 / 0xBB67AE85.  out[4] for
 * counter ctr[4] and key key[2]. */
void glo_philox4x32(const uint32_t* ctr, const uint32_t* key, uint32_t* out) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    c1 = (uint32_t)p1;
    c3 = (uint32_t)p0;
    c0 = n0;
    c2 = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0, out[1] = c1, out[2] = c2, out[3] = c3;
}

/* Triton's tl.randint(seed, offset) (triton/language/random.py, Triton 3.6: randint4x puts the
 * 64-bit offset's halves in the counter's first two words, philox keys with the seed's halves) */
uint32_t glo_randint(uint64_t seed, uint64_t offset) {
  const uint32_t ctr[4] = {(uint32_t)offset, (uint32_t)(offset >> 32), 0u, 0u};
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t out[4];
  glo_philox4x32(ctr, key, out);
  return out[0];
}

static inline uint16_t f32_bits_hi(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)(u >> 16);
}

/* AdamW of bf16 parameters (sparse_pooling/optim.py:26-64): p holds bf16 bits.  With master (fp32,
 * updated in place) the update runs on the master and p = RNE(master) (HAS_MASTER); otherwise on
 * float(p), then p = RNE(p) or, with stochastic, the stochastic rounding of optim.py:59-62:
 * bits(p) + (randint(seed, i) & 0xFFFF), truncated to bf16.  Moments as in glo_adam_f32. */
void glo_adam_bf16(long n, uint16_t* p, float* master, float* g, float* m, float* v, float lr, float b1, float b2,
                   float eps, float wd, float bc1, float bc2, int moments_bf16, int stochastic, uint64_t seed) {
  for (long i = 0; i < n; ++i) {
    float gi = g[i];
    float mi = b1 * m[i] + (1.0f - b1) * gi;
    float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
    float upd = (mi / bc1) / (sqrtf(vi / bc2) + eps);
    uint32_t pb = (uint32_t)p[i] << 16;
    float p0;
    memcpy(&p0, &pb, 4);
    if (master) p0 = master[i];
    float pi = p0 * (1.0f - lr * wd) - lr * upd;
    m[i] = moments_bf16 ? bf16_round(mi) : mi;
    v[i] = moments_bf16 ? bf16_round(vi) : vi;
    g[i] = 0.0f;
    if (master) {
      master[i] = pi;
      p[i] = f32_bits_hi(bf16_round(pi));
    } else if (stochastic) {
      uint32_t u;
      memcpy(&u, &pi, 4);
      u = (u + (glo_randint(seed, (uint64_t)i) & 0xFFFFu)) & 0xFFFF0000u;
      p[i] = (uint16_t)(u >> 16);
    } else {
      p[i] = f32_bits_hi(bf16_round(pi));
    }
  }
}

/* ---- smooth pooling (pools 4, 5, 6) --------------------------------------------------------- */
static inline double smooth_scale(int pool, double param) {
  return pool == 4 ? 1.4426950408889634 / param : (pool == 6 ? 1.4426950408889634 * param : 1.0);
}

/* pooled value, L2 and the pool's largest |u| (LME / softmax) or a (power) of token row xb; z[] [n_g] */
static void smooth_pool(const double* z, int n_g, int act, int pool, double param, double* pre, double* L2,
                        double* amax) {
  if (pool == 5) {
    double M = 0.0;
    for (int s = 0; s < n_g; ++s) M = fmax(M, act_f(z[s], 1));
    double acc = 0.0;
    if (M > 0.0)
      for (int s = 0; s < n_g; ++s) acc += pow(act_f(z[s], 1) / M, param);
    *pre = M > 0.0 ? M * pow(acc / (double)n_g, 1.0 / param) : 0.0;
    *L2 = 0.0;
    *amax = M;
    return;
  }
  const double sc = smooth_scale(pool, param);
  double M = -INFINITY, am = 0.0;
  for (int s = 0; s < n_g; ++s) {
    M = fmax(M, act_f(z[s], act) * sc);
    am = fmax(am, fabs(act_f(z[s], act)));
  }
  double S = 0.0, T = 0.0;
  for (int s = 0; s < n_g; ++s) {
    const double a = act_f(z[s], act), e = exp2(a * sc - M);
    S += e;
    T += e * a;
  }
  *L2 = M + log2(S);
  *pre = pool == 4 ? (*L2 - log2((double)n_g)) / sc : T / S;
  *amax = am;
}

/*
 * Smooth pooling forward.  pre [B, G]; lse [B, G] (optional) the log2-normaliser L2 (0 for
 * power); mag [B, G] (optional): the scale of an fp32 evaluation's error: |pre| + the pool's
 * largest |a| + the largest sum_k |x w| + |bias| of its neurons, times (1 + beta * spread) for
 * softmax-weighted and (M / pre)^(p - 1) for power.
 */
void glo_forward_smooth_f64(int B, int D, int G, int S, int K, const float* x, const int32_t* idx, const float* w,
                            const float* bias, const int32_t* counts, int act, int pool, double param, double* pre,
                            double* lse, double* mag) {
  double* z = (double*)malloc(sizeof(double) * (size_t)S);
  for (int b = 0; b < B; ++b) {
    const float* xb = x + (size_t)b * D;
    for (int g = 0; g < G; ++g) {
      const int n_g = counts[g];
      double zmax = 0.0, zm;
      for (int s = 0; s < n_g; ++s) {
        z[s] = neuron_z(xb, idx, w, bias, (long)g * S + s, K, &zm);
        zmax = fmax(zmax, zm);
      }
      double P, L2, am;
      smooth_pool(z, n_g, act, pool, param, &P, &L2, &am);
      pre[(size_t)b * G + g] = P;
      if (lse) lse[(size_t)b * G + g] = L2;
      if (mag) {
        double amp = 1.0;
        if (pool == 6) amp = 1.0 + param * 2.0 * am;
        if (pool == 5) amp = P > 0.0 ? pow(am / P, param - 1.0) : 1.0;
        mag[(size_t)b * G + g] = fabs(P) + am + zmax * amp;
      }
    }
  }
  free(z);
}

/* Smooth pooling backward (dW, db, dX accumulated in float64, with the sum of |terms| scales). */
void glo_backward_smooth_f64(int B, int D, int G, int S, int K, const float* x, const int32_t* idx, const float* w,
                             const float* bias, const int32_t* counts, int act, int pool, double param, const float* dy,
                             double* dW, double* db, double* dX, double* magW, double* magb, double* magX) {
  double* z = (double*)malloc(sizeof(double) * (size_t)S);
  const double sc = smooth_scale(pool, param);
  for (int b = 0; b < B; ++b) {
    const float* xb = x + (size_t)b * D;
    for (int g = 0; g < G; ++g) {
      const int n_g = counts[g];
      for (int s = 0; s < n_g; ++s) z[s] = neuron_z(xb, idx, w, bias, (long)g * S + s, K, NULL);
      double P, L2, am;
      smooth_pool(z, n_g, act, pool, param, &P, &L2, &am);
      const double g_pre = (double)dy[(size_t)b * G + g];
      for (int s = 0; s < n_g; ++s) {
        double dz;
        if (pool == 5) {
          const double a = act_f(z[s], 1);
          dz = (P > 0.0 && z[s] > 0.0) ? g_pre / (double)n_g * pow(a / P, param - 1.0) : 0.0;
        } else {
          const double a = act_f(z[s], act), pw = exp2(a * sc - L2);
          dz = g_pre * pw * (pool == 6 ? 1.0 + param * (a - P) : 1.0) * dact_f(z[s], act);
        }
        const long n = (long)g * S + s;
        db[n] += dz;
        if (magb) magb[n] += fabs(dz);
        for (int k = 0; k < K; ++k) {
          const int d = idx[n * K + k];
          dW[n * K + k] += dz * (double)xb[d];
          dX[(size_t)b * D + d] += dz * (double)w[n * K + k];
          if (magW) magW[n * K + k] += fabs(dz * (double)xb[d]);
          if (magX) magX[(size_t)b * D + d] += fabs(dz * (double)w[n * K + k]);
        }
      }
    }
  }
  free(z);
}

