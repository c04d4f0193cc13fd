// Max / top-k mean pooling backward as selection events, without floating-point atomics.
//
// Max pooling gives a gradient only to the winner of each (token, pool), top-k mean to its kk =
// min(n_g, k) selected neurons: each selected neuron n* = g*S + slot gets dz = coef * act'(z[b, n*])
// with coef = g_pre[b, g] (max) or g_pre[b, g] / kk (top-k), pytorch_reference.py:61-77 through
// autograd.  The reference runs these as an event kernel with fp32 atomics
// (sparse_pooling/kernels/triton_fused.py:478-520 bwd_events_kernel, launched from
// autograd.py:284-295), touching the selected neurons' K edges only.  Here the same events (KPE
// per (token, pool): 1 or k; slot -1 = none) are summed in a fixed order:
//   * max_events_dw_kernel, one workgroup per pool: each token's event recomputes z (K MACs, as
//     the reference does for act'), the pool's events are sorted by (slot, token) in LDS, and the
//     first event of every slot sums that slot's events in token order and adds them to dW and db
//     (one writer per neuron);
//   * max_events_dx_kernel, one workgroup per token: the events' dz * W[n*, k] are summed into
//     dX[b, idx[n*, k]] as 64-bit fixed-point integers (LDS atomics: integer sums do not depend on
//     their order).  A first pass bounds the terms of every input d by the largest |g_pre| *
//     |W[n*, k]| with idx[n*, k] = d and picks that input's power-of-two scale, under which the sum
//     of all G * kpe * K terms stays below 2^62; the result is converted back once per input.
#include "gl_common.h"
#include "gl_internal.h"

namespace gl {

struct MaxEvK {
  const float4* __restrict__ xt;      // [n_tiles][D] token tiles of the chunk (fp32)
  const int32_t* __restrict__ idx;    // [G*S, K]
  const float* __restrict__ W;        // [G*S, K]
  const float* __restrict__ bias;     // [G*S]
  const int32_t* __restrict__ counts; // [G]
  const float* __restrict__ c1t;      // [G][cap] coef of the chunk's tokens (g_pre, / kk for top-k)
  const int32_t* __restrict__ wint;   // [G][cap][kpe] selected slots of the chunk's tokens
  const float* __restrict__ g_pre;    // [B, G]
  const int32_t* __restrict__ winner; // [B, G, kpe]
  float* dW;                          // [G*S, K] accumulated
  float* db;                          // [G*S] accumulated
  float* dX;                          // [B, D] overwritten
  int D, G, S, cap, Bc, b0, npow2, kpe, tsub;
  int rs;     // log2 slots per shared index record
  bool topk;  // coef = g_pre / min(n_g, kpe)
  int sps, gs;  // pool geometry (pool_base)
  int dblk;     // dX: inputs per block (D when the token's row, bounds and accumulators fit the LDS)
  int wbf;      // W and bias stored as bf16 (widened in the kernel)
};

// x[b, d] of the chunk's token b from the token tiles
__device__ __forceinline__ float tile_x(const float4* xt, int D, int b, int d) {
  const float* e = reinterpret_cast<const float*>(xt + (long long)(b >> 2) * D + d);
  return e[b & 3];
}

// dz of the event (token b, pool g, slot s): g_pre * act'(z), z = bias + sum_k x[idx] w in k order
// W and bias in their stored dtype, chosen at compile time (ld_param_t: a run-time dtype test
// inside the event loops doubled the dX pass)
template <int K, int ACT, bool WBF, typename XF>
__device__ __forceinline__ float event_dz(const MaxEvK& p, long long n, float c1, XF xat, float (&xk)[K],
                                          float (&wk)[K], int (&dk)[K]) {
  float z = ld_param_t<WBF>(p.bias, n);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    int d = rec_index(p.idx, n, k, K, p.rs);
    d = d < 0 ? 0 : (d >= p.D ? p.D - 1 : d);  // host validates; clamp keeps reads in bounds
    dk[k] = d;
    wk[k] = ld_param_t<WBF>(p.W, n * K + k);
    xk[k] = xat(d);
    z = __builtin_fmaf(xk[k], wk[k], z);
  }
  if constexpr (ACT == GL_ACT_GELU) return c1 * dact_f<ACT>(z);
  return ACT == GL_ACT_RELU ? (z > 0.f ? c1 : 0.f) : c1;
}

// dW / db of one pool's events, tsub tokens (tsub * kpe <= 1024 events) at a time.  LDS: npow2
// sort keys, then per event its dz and K products.
template <int K, int ACT, bool WBF>
__global__ void __launch_bounds__(256) max_events_dw_kernel(MaxEvK p) {
  extern __shared__ unsigned lds[];
  unsigned* keys = lds;
  float* ev = reinterpret_cast<float*>(lds + p.npow2);  // [tsub * kpe][K + 1]: dz, dz * x_k
  const int g = blockIdx.x;
  for (int t0 = 0; t0 < p.Bc; t0 += p.tsub) {
    const int nev = (p.Bc - t0 < p.tsub ? p.Bc - t0 : p.tsub) * p.kpe;
    for (int i = threadIdx.x; i < p.npow2; i += blockDim.x) {
      unsigned key = ~0u;  // no event
      if (i < nev) {
        const int bl = t0 + i / p.kpe;  // token of the chunk
        const int s = p.wint[((long long)g * p.cap + bl) * p.kpe + i % p.kpe];
        if (s >= 0 && s < pool_ext(g, p.S, p.sps, p.gs)) {
          const long long n = pool_base(g, p.S, p.sps, p.gs) + s;
          float xk[K], wk[K];
          int dk[K];
          const float dz = event_dz<K, ACT, WBF>(p, n, p.c1t[(long long)g * p.cap + bl],
                                            [&](int d) { return tile_x(p.xt, p.D, bl, d); }, xk, wk, dk);
          float* e = ev + (long long)i * (K + 1);
          e[0] = dz;
#pragma unroll
          for (int k = 0; k < K; ++k) e[1 + k] = dz * xk[k];
          key = ((unsigned)s << 11) | (unsigned)i;  // slot, then event (token-major; i < 1024 < 2^11)
        }
      }
      keys[i] = key;
    }
    __syncthreads();
    for (int size = 2; size <= p.npow2; size <<= 1) {  // bitonic sort, ascending
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = threadIdx.x; i < p.npow2 / 2; i += blockDim.x) {
          const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
          const bool asc = (lo & size) == 0;
          const unsigned a = keys[lo], b = keys[hi];
          if ((a > b) == asc) keys[lo] = b, keys[hi] = a;
        }
        __syncthreads();
      }
    }
    // the first event of each slot sums the slot's events in token order (a neuron is selected at
    // most once per token)
    for (int i = threadIdx.x; i < nev; i += blockDim.x) {
      const unsigned key = keys[i];
      const unsigned s = key >> 11;
      if (key == ~0u || (i > 0 && (keys[i - 1] >> 11) == s)) continue;
      float acc[K + 1];
#pragma unroll
      for (int k = 0; k <= K; ++k) acc[k] = 0.f;
      for (int j = i; j < nev && keys[j] != ~0u && (keys[j] >> 11) == s; ++j) {
        const float* e = ev + (long long)(keys[j] & 2047u) * (K + 1);
#pragma unroll
        for (int k = 0; k <= K; ++k) acc[k] += e[k];
      }
      const long long n = pool_base(g, p.S, p.sps, p.gs) + s;
      p.db[n] += acc[0];
#pragma unroll
      for (int k = 0; k < K; ++k) p.dW[n * K + k] += acc[1 + k];
    }
    __syncthreads();  // the next token group reuses the LDS
  }
}

// 2^e as a double for a power e kept in the normal range
__device__ __forceinline__ double pow2(int e) {
  e = e > 1000 ? 1000 : (e < -1000 ? -1000 : e);
  return __longlong_as_double((long long)(1023 + e) << 52);
}

// dX of one token, its inputs in blocks of dblk (the whole row when it fits the LDS).  The events'
// terms dz * W[n*, k] are summed into dX[b, idx] as fixed-point integers, so the sum does not
// depend on the order of the LDS atomics.  One scale per token, 2^sh with
// sh = 61 - floor(log2(bound)) + 32 for bound = (largest |g_pre| * |W| of the token's events) *
// G * kpe * K: a term t = dz * w * 2^sh (|t| < 2^94, 24 significant bits) splits exactly into
// t = hi * 2^32 + lo (hi = floor(t / 2^32), 0 <= lo < 2^32), and per input the hi parts and the lo
// parts are summed in two 64-bit words (|sum hi| < 2^63; sum lo < 2^32 * 2^31 terms).  The
// quantum is ~2^-70 of the token's largest term (~2^-38 with one 64-bit word), so inputs fed only
// by terms many orders below it keep fp32 accuracy.  LDS: dblk pairs of words, then, with a single
// block, the token's X row (with several, x is read from the token tile in global memory).
template <int K, int ACT, bool ONE, bool WBF>
__global__ void __launch_bounds__(1024) max_events_dx_kernel(MaxEvK p) {
  // ONE is a compile-time choice, so each instantiation reads X from one address space (a run-time
  // choice between the LDS row and the global tile makes the compiler use flat loads for both)
  extern __shared__ unsigned long long ldsq[];
  __shared__ unsigned tokmax;
  const int DB = ONE ? p.D : p.dblk;
  unsigned long long* acc_hi = ldsq;                          // [DB]
  unsigned long long* acc_lo = ldsq + DB;                     // [DB]
  float* xrow = reinterpret_cast<float*>(ldsq + 2 * DB);      // [D], single block only
  const int b = blockIdx.x;
  const long long row = (long long)(p.b0 + b) * p.G;  // [B, G] row of the token; winners: row * kpe
  if constexpr (ONE)
    for (int d = threadIdx.x; d < p.D; d += blockDim.x) xrow[d] = tile_x(p.xt, p.D, b, d);
  if (threadIdx.x == 0) tokmax = 0u;
  __syncthreads();
  // pass 1: every term |dz * W[n*, k]| is at most |g_pre| * |W[n*, k]| * max |act'| (1 for
  // identity and relu, < 1.13 for GELU, bounded by 2 below); the bits of non-negative floats order
  // like the values, so an integer maximum is the float maximum
  float m = 0.f;
  for (int e = threadIdx.x; e < p.G * p.kpe; e += blockDim.x) {
    const int g = e / p.kpe;
    const int s = p.winner[row * p.kpe + e];
    if (s < 0 || s >= pool_ext(g, p.S, p.sps, p.gs)) continue;
    const long long n = pool_base(g, p.S, p.sps, p.gs) + s;
    float wm = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k) wm = __builtin_fmaxf(wm, __builtin_fabsf(ld_param_t<WBF>(p.W, n * K + k)));
    m = __builtin_fmaxf(m, __builtin_fabsf(p.g_pre[row + g]) * wm);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, off));
  if ((threadIdx.x & 63) == 0) atomicMax(&tokmax, __float_as_uint(m));
  __syncthreads();
  const double bound = (double)__uint_as_float(tokmax) * ((double)p.G * (double)p.kpe * (double)K) *
                       (ACT == GL_ACT_GELU ? 2.0 : 1.0);
  const int e2 = bound > 0.0 ? (int)((__double_as_longlong(bound) >> 52) & 0x7ff) - 1023 : 0;
  const int sh = 61 - e2 + 32;
  const double scale = pow2(sh), unscale = pow2(-sh);
  const double two32 = 4294967296.0, inv32 = 1.0 / 4294967296.0;
  for (int lo = 0; lo < p.D; lo += DB) {
    const int nb = p.D - lo < DB ? p.D - lo : DB;
    for (int i = threadIdx.x; i < nb; i += blockDim.x) {
      acc_hi[i] = 0ull;
      acc_lo[i] = 0ull;
    }
    __syncthreads();
    // pass 2: the events' terms, split into (hi, lo) words
    for (int e = threadIdx.x; e < p.G * p.kpe; e += blockDim.x) {
      const int g = e / p.kpe;
      int s = p.winner[row * p.kpe + e];
      const bool ok = s >= 0 && s < pool_ext(g, p.S, p.sps, p.gs);
      s = ok ? s : 0;
      const long long n = pool_base(g, p.S, p.sps, p.gs) + s;
      float xk[K], wk[K];
      int dk[K];
      float coef = p.g_pre[row + g];
      if (p.topk) {  // the same expression as c1t_kernel's
        const int n_g = p.counts[g];
        coef = coef / (float)(n_g < p.kpe ? n_g : p.kpe);
      }
      const float dz = event_dz<K, ACT, WBF>(
          p, n, coef,
          [&](int d) {
            if constexpr (ONE) return xrow[d];
            else return tile_x(p.xt, p.D, b, d);
          },
          xk, wk, dk);
      if (!ok || dz == 0.f) continue;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int i = dk[k] - lo;
        if ((unsigned)i >= (unsigned)nb) continue;
        const double t = __builtin_rint((double)(dz * wk[k]) * scale);  // an integer (exact above 2^24)
        const double h = __builtin_floor(t * inv32);                     // <= 24 significant bits
        const double l = t - h * two32;                                  // exact, in [0, 2^32)
        atomicAdd(&acc_hi[i], (unsigned long long)(long long)h);
        atomicAdd(&acc_lo[i], (unsigned long long)(unsigned)l);
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nb; i += blockDim.x) {
      // value = hi * 2^32 + lo, carried in integers first so the one rounding is to double
      const unsigned long long lw = acc_lo[i];
      const long long hw = (long long)acc_hi[i] + (long long)(lw >> 32);
      const double v = ((double)hw * two32 + (double)(unsigned)(lw & 0xffffffffull)) * unscale;
      p.dX[(long long)(p.b0 + b) * p.D + lo + i] = (float)v;
    }
    __syncthreads();  // the next block reinitialises the accumulators
  }
}

template <int K, int ACT, bool WBF>
static int launch_max_events_kw(MaxEvK k, hipStream_t s) {
  const size_t dw_lds = (size_t)k.npow2 * 4 + (size_t)k.tsub * k.kpe * (K + 1) * 4;
  // dX: the whole row (20 bytes per input: two accumulator words and x) when it fits, else blocks
  // of 16-byte inputs (the kernel's static LDS word aside)
  const size_t room = max_lds_bytes() - 64;
  size_t dx_lds = (size_t)k.D * 20;
  k.dblk = k.D;
  if (dx_lds > room) {
    k.dblk = (int)(room / 16 / 64 * 64);
    dx_lds = (size_t)k.dblk * 16;
  }
  if (dw_lds > max_lds_bytes() || k.dblk < 64) return GL_ERR_LDS;
  GL_TRY(set_lds_limit((const void*)max_events_dw_kernel<K, ACT, WBF>, dw_lds));
  const bool one = k.dblk >= k.D;
  const void* dxk = one ? (const void*)max_events_dx_kernel<K, ACT, true, WBF> : (const void*)max_events_dx_kernel<K, ACT, false, WBF>;
  GL_TRY(set_lds_limit(dxk, dx_lds));
  GL_LAUNCH(GL_KERNEL_MAX_EV_DW, (max_events_dw_kernel<K, ACT, WBF>), dim3((unsigned)k.G), dim3(256), dw_lds, s, k);
  GL_CHECK_LAUNCH();
  if (one)
    GL_LAUNCH(GL_KERNEL_MAX_EV_DX, (max_events_dx_kernel<K, ACT, true, WBF>), dim3((unsigned)k.Bc), dim3(1024), dx_lds, s, k);
  else
    GL_LAUNCH(GL_KERNEL_MAX_EV_DX, (max_events_dx_kernel<K, ACT, false, WBF>), dim3((unsigned)k.Bc), dim3(1024), dx_lds, s, k);
  GL_CHECK_LAUNCH();
  return 0;
}

template <int K, int ACT>
static int launch_max_events_k(const MaxEvK& k, hipStream_t s) {
  return k.wbf ? launch_max_events_kw<K, ACT, true>(k, s) : launch_max_events_kw<K, ACT, false>(k, s);
}

int launch_max_events(int K, int act, const MaxEvKArgs& a, hipStream_t s) {
  // tokens per dW sort: at most 1024 events (the sort keys hold the event index in 11 bits)
  const int tsub = a.Bc < 1024 / a.kpe ? a.Bc : 1024 / a.kpe;
  int npow2 = 1;
  while (npow2 < tsub * a.kpe) npow2 <<= 1;
  const MaxEvK k{a.xt, a.idx, a.W, a.bias, a.counts, a.c1t, a.wint, a.g_pre, a.winner, a.dW, a.db, a.dX,
                 a.D, a.G, a.S, a.cap, a.Bc, a.b0, npow2, a.kpe, tsub, a.rs, a.topk, a.sps, a.gs, a.D, a.wbf};
  if (act == GL_ACT_GELU) return K == 8 ? launch_max_events_k<8, GL_ACT_GELU>(k, s) : launch_max_events_k<16, GL_ACT_GELU>(k, s);
  if (K == 8) return act == GL_ACT_RELU ? launch_max_events_k<8, GL_ACT_RELU>(k, s) : launch_max_events_k<8, GL_ACT_IDENTITY>(k, s);
  return act == GL_ACT_RELU ? launch_max_events_k<16, GL_ACT_RELU>(k, s) : launch_max_events_k<16, GL_ACT_IDENTITY>(k, s);
}

}  // namespace gl
