// Backward: recompute z, then dW/db (per-edge reduction over the batch) and dX (deterministic
// segmented reduction over the input-major edge list).  No floating-point atomics.
//
// Pass 1 (bwd_w_kernel) is neuron-stationary like the forward: a wave keeps its chunk's
// parameters and dW/db accumulators in VGPRs and streams the token tiles through LDS.  Per
// (token, neuron) it recomputes z, forms dz = c1[b, g] * act'(z) (ops.py:242-249 mean:
// c1 = g_pre / n_g; sum: c1 = g_pre), accumulates db += dz and dW[k] += dz * x_k in token order,
// and records the activation mask bit act'(z) of every token (a [neurons, tokens] bit matrix, 1/32
// of the bytes of the fp32 hidden tensor).  At the end it adds dW/db to the caller's accumulators.
//
// Pass 2 (dx_kernel) owns 16 consecutive input features, one pool range and 64*T tokens per
// wave.  It walks the input-major edges of its features in the fixed order (unit, feature, edge
// id); for every edge (n, k) it adds c1[b, g(n)] * W[n,k] * mask[n, b] to the register
// accumulator of its feature.  The pool-range partials are summed in a fixed order by
// dx_reduce_kernel.  Reference: _bwd_tile Mode A (sparse_pooling/kernels/triton_fused.py:402-445),
// which uses fp32 atomics for dW and dX instead.
#include "gl_common.h"
#include "gl_internal.h"

namespace gl {

// c1t[g, b] = g_pre[b0 + b, g] * scale_g for b < Bc, zero up to cap (tiled transpose).
__global__ void __launch_bounds__(256) c1t_kernel(const float* __restrict__ g_pre, const int32_t* __restrict__ counts,
                                                  float* __restrict__ c1t, int G, int b0, int Bc, int cap, int pool) {
  __shared__ float tile[32][33];
  const int g0 = blockIdx.x * 32, bb = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int r = ty; r < 32; r += 8) {
    const int b = bb + r, g = g0 + tx;
    tile[r][tx] = (b < Bc && g < G) ? g_pre[(long long)(b0 + b) * G + g] : 0.f;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int g = g0 + r, b = bb + tx;
    if (g < G && b < cap) {
      float v = tile[tx][r];
      if (pool == GL_POOL_MEAN) v = v / (float)counts[g];
      c1t[(long long)g * cap + b] = v;
    }
  }
}

struct BwK {
  const float4* __restrict__ xt;
  const int32_t* __restrict__ idx;
  const float* __restrict__ W;
  const float* __restrict__ bias;
  const int32_t* __restrict__ counts;
  const float* __restrict__ c1t;
  float* dW;
  float* db;
  uint32_t* mask;  // [G*S][rs] activation-mask words
  long long n_chunks;
  int D, S, cpg, n_tiles, cap, rs;
};

template <int K, int NPL, int WAVES, int ACT, int PF>
__global__ void __launch_bounds__(WAVES * 64) bwd_w_kernel(BwK p) {
  extern __shared__ float4 xs[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  long long chunk = (long long)blockIdx.x * WAVES + wave;
  const bool active = chunk < p.n_chunks;
  if (!active) chunk = p.n_chunks - 1;  // idle waves of the last block recompute a real chunk, store nothing
  const long long g = chunk / p.cpg;
  const int s_lo = (int)(chunk % p.cpg) * 64 * NPL;
  const int n_g = p.counts[g];

  unsigned addr[NPL][K];
  float w[NPL][K], dw[NPL][K];
  float bias[NPL], dbv[NPL];
  unsigned mw[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int s = s_lo + j * 64 + lane;
    const bool valid = s < n_g;
    const long long n = g * p.S + (s < p.S ? s : p.S - 1);  // in-bounds address; invalid slots masked
#pragma unroll
    for (int k = 0; k < K; ++k) {
      int d = p.idx[n * K + k];
      d = (d < 0 || !valid) ? 0 : (d >= p.D ? p.D - 1 : d);  // host validates; clamp keeps LDS reads in bounds
      addr[j][k] = (unsigned)d * 16u;
      const float wl = p.W[n * K + k];
      w[j][k] = valid ? wl : 0.f;
      dw[j][k] = 0.f;
    }
    const float bl = p.bias[n];
    bias[j] = valid ? bl : 0.f;
    dbv[j] = 0.f;
    mw[j] = 0u;
  }
  const float* c1row = p.c1t + g * p.cap;
  const char* xsb = reinterpret_cast<const char*>(xs);
  // token tiles are staged as in the forward (PF > 0: next tile prefetched into registers)
  constexpr int NT = WAVES * 64;
  PrefetchRegs<PF> pf;
  if constexpr (PF > 0) pf.load(p.xt, NT);

  // 8 token tiles (32 tokens) per mask word; the word is stored after the inner loop
  for (int t0 = 0; t0 < p.n_tiles; t0 += 8) {
    unsigned mw[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) mw[j] = 0u;
    const int t1 = t0 + 8 < p.n_tiles ? t0 + 8 : p.n_tiles;
    for (int t = t0; t < t1; ++t) {
      __syncthreads();
      if constexpr (PF > 0) {
        pf.store(xs, NT);
      } else {
        const float4* src = p.xt + (long long)t * p.D;
        for (int i = threadIdx.x; i < p.D; i += NT) xs[i] = src[i];
      }
      __syncthreads();
      const float4 c1 = *reinterpret_cast<const float4*>(c1row + t * BT);  // issued before the prefetch
      if constexpr (PF > 0) {
        if (t + 1 < p.n_tiles) pf.load(p.xt + (long long)(t + 1) * p.D, NT);
      }
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        float4 x[K];
        float z0 = bias[j], z1 = bias[j], z2 = bias[j], z3 = bias[j];
#pragma unroll
        for (int k = 0; k < K; ++k) {
          x[k] = *reinterpret_cast<const float4*>(xsb + addr[j][k]);
          z0 = __builtin_fmaf(x[k].x, w[j][k], z0);
          z1 = __builtin_fmaf(x[k].y, w[j][k], z1);
          z2 = __builtin_fmaf(x[k].z, w[j][k], z2);
          z3 = __builtin_fmaf(x[k].w, w[j][k], z3);
        }
        const bool m0 = ACT != GL_ACT_RELU || z0 > 0.f, m1 = ACT != GL_ACT_RELU || z1 > 0.f;
        const bool m2 = ACT != GL_ACT_RELU || z2 > 0.f, m3 = ACT != GL_ACT_RELU || z3 > 0.f;
        const float d0 = m0 ? c1.x : 0.f, d1 = m1 ? c1.y : 0.f, d2 = m2 ? c1.z : 0.f, d3 = m3 ? c1.w : 0.f;
        dbv[j] = dbv[j] + d0 + d1 + d2 + d3;
#pragma unroll
        for (int k = 0; k < K; ++k) {
          float a = dw[j][k];
          a = __builtin_fmaf(d0, x[k].x, a);
          a = __builtin_fmaf(d1, x[k].y, a);
          a = __builtin_fmaf(d2, x[k].z, a);
          a = __builtin_fmaf(d3, x[k].w, a);
          dw[j][k] = a;
        }
        mw[j] |= ((unsigned)m0 | ((unsigned)m1 << 1) | ((unsigned)m2 << 2) | ((unsigned)m3 << 3)) << ((t & 7) * 4);
        // keeps the gathers of the unrolled neuron loop from all being hoisted (register pressure)
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    const int ln = opaque(lane);  // address math kept local (see opaque())
    uint32_t* mrow = p.mask + (g * p.S + s_lo + ln) * p.rs + (t0 >> 3);
#pragma unroll
    for (int j = 0; j < NPL; ++j)
      if (active && s_lo + j * 64 + ln < n_g) mrow[(long long)j * 64 * p.rs] = mw[j];
  }
  if (!active) return;
  const int words_written = (p.n_tiles + 7) >> 3;
  const int ln = opaque(lane);
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int s = s_lo + j * 64 + ln;
    if (s >= n_g) continue;
    const long long n = g * p.S + s;
#pragma unroll
    for (int k = 0; k < K; ++k) p.dW[n * K + k] += dw[j][k];
    p.db[n] += dbv[j];
    uint32_t* r = p.mask + n * p.rs;
    for (int wi = words_written; wi < p.rs; ++wi) r[wi] = 0u;  // tokens of the padded chunk tail
  }
}

struct DxK {
  const uint32_t* __restrict__ rec;
  const uint32_t* __restrict__ seg_ptr;
  const int32_t* __restrict__ seg_unit;
  const uint32_t* __restrict__ seg_begin;
  const float* __restrict__ c1t;
  const uint32_t* __restrict__ mask;
  const float* __restrict__ W;
  float* part;  // [Q][D][cap]
  int D, S, K, P, U, Q, UQ, cap, rs, n_tc;
};

// Edges are consumed in batches of DX_BATCH.  One inline-assembly block requests, with scalar
// loads, the weight and the T 64-bit mask words of every edge of the batch plus the records of
// the next batch, then waits once: a wave pays one memory round trip per batch, and the loads,
// the wait and the destination registers sit in one statement so no compiler-inserted copy can
// read a register before its load has landed.  The edges of one unit segment come sorted by
// feature; a register run accumulates consecutive edges of one feature and is added to that
// feature's accumulator -- a lane-private LDS column, so the feature index may vary at run time --
// when the feature changes.
constexpr int DX_BATCH = 4;

template <int T>
struct MaskWords;
template <>
struct MaskWords<1> {
  typedef unsigned __attribute__((ext_vector_type(2))) v;
};
template <>
struct MaskWords<2> {
  typedef unsigned __attribute__((ext_vector_type(4))) v;
};
template <>
struct MaskWords<4> {
  typedef unsigned __attribute__((ext_vector_type(8))) v;
};
typedef unsigned __attribute__((ext_vector_type(4))) u32x4;

#define GL_SLOAD_MASK(T) (T == 1 ? "s_load_dwordx2" : (T == 2 ? "s_load_dwordx4" : "s_load_dwordx8"))

template <int T>
__device__ __forceinline__ void dx_batch_loads(const float* w0, const float* w1, const float* w2, const float* w3,
                                               const void* m0p, const void* m1p, const void* m2p, const void* m3p,
                                               const void* recp, float (&w)[DX_BATCH],
                                               typename MaskWords<T>::v (&m)[DX_BATCH], u32x4& rec) {
  unsigned wb0, wb1, wb2, wb3;
  if constexpr (T == 1) {
    asm volatile(
        "s_load_dword %0, %9, 0x0\n s_load_dword %1, %10, 0x0\n s_load_dword %2, %11, 0x0\n"
        "s_load_dword %3, %12, 0x0\n s_load_dwordx2 %4, %13, 0x0\n s_load_dwordx2 %5, %14, 0x0\n"
        "s_load_dwordx2 %6, %15, 0x0\n s_load_dwordx2 %7, %16, 0x0\n s_load_dwordx4 %8, %17, 0x0\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(wb0), "=&s"(wb1), "=&s"(wb2), "=&s"(wb3), "=&s"(m[0]), "=&s"(m[1]), "=&s"(m[2]), "=&s"(m[3]),
          "=&s"(rec)
        : "s"(w0), "s"(w1), "s"(w2), "s"(w3), "s"(m0p), "s"(m1p), "s"(m2p), "s"(m3p), "s"(recp)
        : "memory");
  } else if constexpr (T == 2) {
    asm volatile(
        "s_load_dword %0, %9, 0x0\n s_load_dword %1, %10, 0x0\n s_load_dword %2, %11, 0x0\n"
        "s_load_dword %3, %12, 0x0\n s_load_dwordx4 %4, %13, 0x0\n s_load_dwordx4 %5, %14, 0x0\n"
        "s_load_dwordx4 %6, %15, 0x0\n s_load_dwordx4 %7, %16, 0x0\n s_load_dwordx4 %8, %17, 0x0\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(wb0), "=&s"(wb1), "=&s"(wb2), "=&s"(wb3), "=&s"(m[0]), "=&s"(m[1]), "=&s"(m[2]), "=&s"(m[3]),
          "=&s"(rec)
        : "s"(w0), "s"(w1), "s"(w2), "s"(w3), "s"(m0p), "s"(m1p), "s"(m2p), "s"(m3p), "s"(recp)
        : "memory");
  } else {
    asm volatile(
        "s_load_dword %0, %9, 0x0\n s_load_dword %1, %10, 0x0\n s_load_dword %2, %11, 0x0\n"
        "s_load_dword %3, %12, 0x0\n s_load_dwordx8 %4, %13, 0x0\n s_load_dwordx8 %5, %14, 0x0\n"
        "s_load_dwordx8 %6, %15, 0x0\n s_load_dwordx8 %7, %16, 0x0\n s_load_dwordx4 %8, %17, 0x0\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(wb0), "=&s"(wb1), "=&s"(wb2), "=&s"(wb3), "=&s"(m[0]), "=&s"(m[1]), "=&s"(m[2]), "=&s"(m[3]),
          "=&s"(rec)
        : "s"(w0), "s"(w1), "s"(w2), "s"(w3), "s"(m0p), "s"(m1p), "s"(m2p), "s"(m3p), "s"(recp)
        : "memory");
  }
  w[0] = __uint_as_float(wb0);
  w[1] = __uint_as_float(wb1);
  w[2] = __uint_as_float(wb2);
  w[3] = __uint_as_float(wb3);
}

template <int T>
__global__ void __launch_bounds__(64) dx_kernel(DxK p) {
  __shared__ float acc[FW][T][64];  // lane-private columns: no barrier needed
  const int lane = threadIdx.x;
  const int bid = blockIdx.x;
  const int tc = bid % p.n_tc;
  const int q = (bid / p.n_tc) % p.Q;
  const int F = bid / (p.n_tc * p.Q);
  const int u_lo = q * p.UQ;
  const int u_hi = min(u_lo + p.UQ, p.U);
  // segments of feature range F whose unit lies in [u_lo, u_hi) (units ascend within F)
  int lo = (int)p.seg_ptr[F], hi = (int)p.seg_ptr[F + 1];
  {
    int a = lo, b = hi;
    while (a < b) {
      int m = (a + b) >> 1;
      if (p.seg_unit[m] < u_lo) a = m + 1; else b = m;
    }
    lo = a;
    b = hi;
    while (a < b) {
      int m = (a + b) >> 1;
      if (p.seg_unit[m] < u_hi) a = m + 1; else b = m;
    }
    hi = a;
  }
#pragma unroll
  for (int f = 0; f < FW; ++f)
#pragma unroll
    for (int j = 0; j < T; ++j) acc[f][j][lane] = 0.f;

  const int tok0 = tc * 64 * T + lane;
  const uint32_t* mask_tc = p.mask + (long long)tc * 2 * T;  // this wave's 64-bit words of every record
  for (int si = lo; si < hi; ++si) {
    const int u = p.seg_unit[si];
    const unsigned e0 = p.seg_begin[si];
    const unsigned e1 = p.seg_begin[si + 1];
    const long long g = u / p.P;
    const long long nb = g * p.S + (long long)(u % p.P) * US;
    float c1[T];
#pragma unroll
    for (int j = 0; j < T; ++j) c1[j] = p.c1t[g * p.cap + tok0 + j * 64];
    float run[T];
#pragma unroll
    for (int j = 0; j < T; ++j) run[j] = 0.f;
    // records of the first batch (the record array carries DX_BATCH entries of padding)
    const u32x4 r0 = *reinterpret_cast<const u32x4*>(p.rec + e0);
    unsigned r[DX_BATCH] = {r0[0], r0[1], r0[2], r0[3]};
    int fcur = (int)(r[0] >> (REC_N_BITS + REC_K_BITS));
    for (unsigned e = e0; e < e1; e += DX_BATCH) {
      const float* wp[DX_BATCH];
      const void* mp[DX_BATCH];
#pragma unroll
      for (int i = 0; i < DX_BATCH; ++i) {
        // past the segment end: reuse the first edge (in bounds; its contribution is skipped)
        const unsigned ri = e + i < e1 ? r[i] : r[0];
        const long long n = nb + (ri & ((1u << REC_N_BITS) - 1));
        const int k = (ri >> REC_N_BITS) & ((1 << REC_K_BITS) - 1);
        wp[i] = p.W + n * p.K + k;
        mp[i] = mask_tc + n * p.rs;
      }
      float wv[DX_BATCH];
      typename MaskWords<T>::v mv[DX_BATCH];
      u32x4 rn;
      dx_batch_loads<T>(wp[0], wp[1], wp[2], wp[3], mp[0], mp[1], mp[2], mp[3], p.rec + e + DX_BATCH, wv, mv, rn);
#pragma unroll
      for (int i = 0; i < DX_BATCH; ++i) {
        if (e + i < e1) {
          const int f = (int)(r[i] >> (REC_N_BITS + REC_K_BITS));
          if (f != fcur) {
#pragma unroll
            for (int j = 0; j < T; ++j) {
              acc[fcur][j][lane] += run[j];
              run[j] = 0.f;
            }
            fcur = f;
          }
#pragma unroll
          for (int j = 0; j < T; ++j) {
            const uint64_t mj = (uint64_t)mv[i][2 * j] | ((uint64_t)mv[i][2 * j + 1] << 32);
            run[j] = __builtin_fmaf(__builtin_amdgcn_inverse_ballot_w64(mj) ? c1[j] : 0.f, wv[i], run[j]);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < DX_BATCH; ++i) r[i] = rn[i];
    }
#pragma unroll
    for (int j = 0; j < T; ++j) acc[fcur][j][lane] += run[j];
  }
  float* out = p.part + (long long)q * p.D * p.cap;
#pragma unroll
  for (int f = 0; f < FW; ++f) {
    const int d = F * FW + f;
    if (d < p.D) {
#pragma unroll
      for (int j = 0; j < T; ++j) out[(long long)d * p.cap + tok0 + j * 64] = acc[f][j][lane];
    }
  }
}

// dX[b0 + b, d] = sum_q part[q, d, b]  (fixed order), tiled transpose to [B, D].
__global__ void __launch_bounds__(256) dx_reduce_kernel(const float* __restrict__ part, float* __restrict__ dX, int D,
                                                        int cap, int Q, int b0, int Bc) {
  __shared__ float tile[32][33];
  const int d0 = blockIdx.x * 32, bb = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int r = ty; r < 32; r += 8) {
    const int d = d0 + r, b = bb + tx;
    float v = 0.f;
    if (d < D && b < Bc) {
      const float* src = part + (long long)d * cap + b;
      for (int q = 0; q < Q; ++q) v += src[(long long)q * D * cap];
    }
    tile[r][tx] = v;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int b = bb + r, d = d0 + tx;
    if (d < D && b < Bc) dX[(long long)(b0 + b) * D + d] = tile[tx][r];
  }
}

// ---- host side -------------------------------------------------------------------------------
struct BwdPlan {
  int bc_max, npl, waves, cpg, tiles_max, cap_max, rs_max, FR, P, U, Q, UQ;
  long long n_chunks, e_max, nseg_max;
  size_t lds, xt_bytes, c1_bytes, mask_bytes, part_bytes, edges_bytes;
};

static BwdPlan bwd_plan(int B, int D, int G, int S, int K) {
  BwdPlan q;
  q.bc_max = B < BWD_TOKEN_CHUNK ? B : BWD_TOKEN_CHUNK;
  q.npl = 48 / K;  // 6 neurons per lane at K = 8, 3 at K = 16
  q.waves = 8;
  q.cpg = ceil_div(S, 64 * q.npl);
  q.n_chunks = (long long)G * q.cpg;
  q.tiles_max = ceil_div(q.bc_max, BT);
  q.cap_max = dx_cap(q.bc_max);
  q.rs_max = mask_stride(q.bc_max);
  q.FR = ceil_div(D, FW);
  q.P = ceil_div(S, US);
  q.U = G * q.P;
  const int n_tc = q.cap_max / (64 * dx_slots(q.bc_max));
  const long long waves_wanted = 8192;
  long long Qw = (waves_wanted + (long long)q.FR * n_tc - 1) / ((long long)q.FR * n_tc);
  if (Qw < 1) Qw = 1;
  if (Qw > q.U) Qw = q.U;
  if (Qw > 64) Qw = 64;
  q.UQ = ceil_div(q.U, Qw);
  q.Q = ceil_div(q.U, q.UQ);
  q.lds = (size_t)D * 16;
  q.xt_bytes = (size_t)round_up((long long)q.tiles_max * D * 16, 256);
  q.c1_bytes = (size_t)round_up((long long)G * q.cap_max * 4, 256);
  q.mask_bytes = (size_t)round_up((long long)G * S * q.rs_max * 4, 256);
  q.part_bytes = (size_t)round_up((long long)q.Q * D * q.cap_max * 4, 256);
  q.e_max = (long long)G * S * K;
  q.nseg_max = (long long)q.FR * q.U < q.e_max ? (long long)q.FR * q.U : q.e_max;
  return q;
}

// byte layout of the edge structure (shared with gl_edges.hip)
void edge_layout(int D, int G, int S, int K, EdgeHeader* h, size_t* total) {
  BwdPlan q = bwd_plan(1, D, G, S, K);
  h->magic = GL_EDGE_MAGIC;
  h->D = D; h->G = G; h->S = S; h->K = K;
  h->fw = FW; h->us = US;
  h->FR = q.FR; h->P = q.P; h->U = q.U;
  size_t off = round_up(sizeof(EdgeHeader), 256);
  h->off_seg_ptr = off;
  off += round_up((q.FR + 1) * 4LL, 256);
  h->off_seg_unit = off;
  off += round_up(q.nseg_max * 4LL, 256);
  h->off_seg_begin = off;
  off += round_up((q.nseg_max + 1) * 4LL, 256);
  h->off_rec = off;
  off += round_up((q.e_max + 8) * 4LL, 256);  // padding: the dX kernel reads records in batches
  *total = off;
}

template <int K, int NPL, int WAVES, int ACT, int PF>
static int launch_bwd_w(const BwK& k, hipStream_t s, size_t lds) {
  auto fn = bwd_w_kernel<K, NPL, WAVES, ACT, PF>;
  GL_TRY(set_lds_limit((const void*)fn, lds));
  GL_LAUNCH(GL_KERNEL_BWD_W, fn, dim3((unsigned)ceil_div(k.n_chunks, WAVES)), dim3(WAVES * 64), lds, s, k);
  GL_CHECK_LAUNCH();
  return 0;
}

// 8 waves per workgroup; next-tile register prefetch when D is a multiple of 512 and needs at
// most MAXPF float4 per thread (the dW accumulators leave no room for more)
template <int ACT, int K, int NPL, int MAXPF>
static int launch_bwd_w_pf(int D, const BwK& k, hipStream_t s, size_t lds) {
  int pf = D % 512 == 0 ? D / 512 : 0;
  if (pf > MAXPF) pf = 0;
  switch (pf) {
    case 1: return launch_bwd_w<K, NPL, 8, ACT, 1>(k, s, lds);
    case 2: return launch_bwd_w<K, NPL, 8, ACT, 2>(k, s, lds);
    case 4: return launch_bwd_w<K, NPL, 8, ACT, 4>(k, s, lds);
    case 8: return launch_bwd_w<K, NPL, 8, ACT, 8>(k, s, lds);
    default: return launch_bwd_w<K, NPL, 8, ACT, 0>(k, s, lds);
  }
}

template <int ACT>
static int launch_bwd_w_act(int K, int D, const BwK& k, hipStream_t s, size_t lds) {
  if (K == 8) return launch_bwd_w_pf<ACT, 8, 6, 8>(D, k, s, lds);
  return launch_bwd_w_pf<ACT, 16, 3, 4>(D, k, s, lds);
}

static int launch_bwd_w_any(int K, int D, int act, const BwK& k, hipStream_t s, size_t lds) {
  return act == GL_ACT_RELU ? launch_bwd_w_act<GL_ACT_RELU>(K, D, k, s, lds)
                            : launch_bwd_w_act<GL_ACT_IDENTITY>(K, D, k, s, lds);
}

static int launch_dx(int T, const DxK& k, int FR, hipStream_t s) {
  dim3 grid((unsigned)((long long)FR * k.Q * k.n_tc));
  switch (T) {
    case 1: GL_LAUNCH(GL_KERNEL_DX, dx_kernel<1>, grid, dim3(64), 0, s, k); break;
    case 2: GL_LAUNCH(GL_KERNEL_DX, dx_kernel<2>, grid, dim3(64), 0, s, k); break;
    default: GL_LAUNCH(GL_KERNEL_DX, dx_kernel<4>, grid, dim3(64), 0, s, k); break;
  }
  GL_CHECK_LAUNCH();
  return 0;
}

}  // namespace gl

using namespace gl;

extern "C" int gl_bwd_workspace(const GlBwdArgs* a, size_t* bytes) {
  if (!a || !bytes) return GL_ERR_ARG;
  GL_TRY(check_layer(a->B, a->D, a->G, a->S, a->K, a->act, a->pool, a->X, a->idx, a->W, a->bias, a->counts,
                     a->x_dtype));
  BwdPlan q = bwd_plan(a->B, a->D, a->G, a->S, a->K);
  *bytes = q.xt_bytes + q.c1_bytes + q.mask_bytes + q.part_bytes;
  return 0;
}

extern "C" int gl_bwd(const GlBwdArgs* a, void* stream) {
  if (!a || !a->g_pre || !a->dW || !a->db || !a->dX || !a->edges) return GL_ERR_ARG;
  size_t need = 0;
  GL_TRY(gl_bwd_workspace(a, &need));
  if (!a->ws || a->ws_bytes < need) return GL_ERR_WORKSPACE;
  EdgeHeader h;
  size_t edge_bytes = 0;
  edge_layout(a->D, a->G, a->S, a->K, &h, &edge_bytes);
  if (a->edges_bytes < edge_bytes) return GL_ERR_EDGES;
  hipStream_t s = (hipStream_t)stream;
  BwdPlan q = bwd_plan(a->B, a->D, a->G, a->S, a->K);
  char* ws = (char*)a->ws;
  float4* xt = (float4*)ws;
  float* c1t = (float*)(ws + q.xt_bytes);
  uint32_t* mask = (uint32_t*)(ws + q.xt_bytes + q.c1_bytes);
  float* part = (float*)(ws + q.xt_bytes + q.c1_bytes + q.mask_bytes);
  const char* eb = (const char*)a->edges;

  for (int b0 = 0; b0 < a->B; b0 += q.bc_max) {
    const int Bc = a->B - b0 < q.bc_max ? a->B - b0 : q.bc_max;
    const int n_tiles = ceil_div(Bc, BT);
    const int T = dx_slots(Bc);
    const int cap = dx_cap(Bc);
    const int rs = mask_stride(Bc);
    GL_TRY(launch_tile_x(a->X, a->sxb, a->x_dtype, a->B, a->D, b0, n_tiles, xt, s));
    GL_LAUNCH(GL_KERNEL_C1T, c1t_kernel, dim3((unsigned)ceil_div(a->G, 32), (unsigned)ceil_div(cap, 32)), dim3(256), 0, s,
                       a->g_pre, a->counts, c1t, a->G, b0, Bc, cap, a->pool);
    GL_CHECK_LAUNCH();
    BwK bk{xt, a->idx, a->W, a->bias, a->counts, c1t, a->dW, a->db, mask, q.n_chunks,
           a->D, a->S, q.cpg, n_tiles, cap, rs};
    GL_TRY(launch_bwd_w_any(a->K, a->D, a->act, bk, s, q.lds));
    DxK dk{(const uint32_t*)(eb + h.off_rec), (const uint32_t*)(eb + h.off_seg_ptr),
           (const int32_t*)(eb + h.off_seg_unit), (const uint32_t*)(eb + h.off_seg_begin), c1t, mask, a->W, part,
           a->D, a->S, a->K, q.P, q.U, q.Q, q.UQ, cap, rs, cap / (64 * T)};
    GL_TRY(launch_dx(T, dk, q.FR, s));
    GL_LAUNCH(GL_KERNEL_DX_REDUCE, dx_reduce_kernel, dim3((unsigned)ceil_div(a->D, 32), (unsigned)ceil_div(Bc, 32)), dim3(256), 0,
                       s, part, a->dX, a->D, cap, q.Q, b0, Bc);
    GL_CHECK_LAUNCH();
  }
  return 0;
}
