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
// Pass 2 (dx_kernel) owns FW = 8 consecutive input features, one unit range and 64*T tokens per
// wave.  It walks the input-major edges of its features in the fixed order (unit, feature, edge
// id); for every edge (n, k) it adds c1[b, g(n)] * W[n,k] * mask[n, b] to the register
// accumulator of its feature.  The pool-range partials are summed in a fixed order by
// dx_reduce_kernel.  Reference: _bwd_tile Mode A (sparse_pooling/kernels/triton_fused.py:402-445),
// which uses fp32 atomics for dW and dX instead.
#include <type_traits>

#include "gl_common.h"
#include "gl_internal.h"

namespace gl {

// c1t[g, b] = g_pre[b0 + b, g] * scale_g for b < Bc, zero up to cap (tiled transpose); scale_g =
// 1 / n_g (mean), 1 / min(n_g, k) (top-k mean), else 1.  Max pooling (winner != null) also
// transposes the winner slots: wint[g, b] = winner[b0 + b, g], -1 up to cap.
__global__ void __launch_bounds__(256) c1t_kernel(const float* __restrict__ g_pre, const int32_t* __restrict__ counts,
                                                  float* __restrict__ c1t, int G, int b0, int Bc, int cap, int pool,
                                                  int topk, const int32_t* __restrict__ winner,
                                                  int32_t* __restrict__ wint) {
  __shared__ float tile[32][33];
  __shared__ int tw[32][33];
  const int g0 = blockIdx.x * 32, bb = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int r = ty; r < 32; r += 8) {
    const int b = bb + r, g = g0 + tx;
    const bool in = b < Bc && g < G;
    tile[r][tx] = in ? g_pre[(long long)(b0 + b) * G + g] : 0.f;
    if (winner) tw[r][tx] = in ? winner[(long long)(b0 + b) * G + g] : -1;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int g = g0 + r, b = bb + tx;
    if (g < G && b < cap) {
      float v = tile[tx][r];
      if (pool == GL_POOL_MEAN) v = v / (float)counts[g];
      if (pool == GL_POOL_TOPK_MEAN) v = v / (float)(counts[g] < topk ? counts[g] : topk);
      c1t[(long long)g * cap + b] = v;
      if (winner) wint[(long long)g * cap + b] = tw[tx][r];
    }
  }
}

// Top-k slots of the chunk's tokens, pool-major: wint[g, b, j] = slots[b0 + b, g, j] (-1 past Bc).
__global__ void __launch_bounds__(256) events_transpose_kernel(const int32_t* __restrict__ slots,
                                                               int32_t* __restrict__ wint, int G, int b0, int Bc,
                                                               int cap, int kpe) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;  // (g, b, j), j fastest
  if (i >= (long long)G * cap * kpe) return;
  const int j = (int)(i % kpe);
  const long long gb = i / kpe;
  const int b = (int)(gb % cap), g = (int)(gb / cap);
  wint[i] = b < Bc ? slots[((long long)(b0 + b) * G + g) * kpe + j] : -1;
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
  uint32_t* mask;  // [n_tc][G*S][mw2] activation-mask words (one slab per dX token slice)
  const uint32_t* sched;  // gather schedule or null
  const uint32_t* win;    // per-pool window starts (window staging) or null
  long long n_chunks, NS;
  int D, S, cpg, n_tiles, cap, mw2, nwin;
  int G, ww, npw;         // window staging: pools, padded window width, pools per workgroup
  int rs;                 // log2 slots per shared index record
  int sps, gs;            // pool geometry (pool_base)
  int tb;                 // tokens per tile: 4, or 2 (two-token tiles; n_tiles counts those)
  int xb;                 // 4-token tiles of raw bf16 (8-byte slots; bf16 X)
  int wbf;                // W and bias stored as bf16 (widened in the kernel)
  const uint16_t* fm;     // the forward's ReLU bits ([n_chunks][fm_tiles][64] 16-bit words) or null
  int fm_tiles, fm_t0;    // 4-token tiles of the whole batch; the backward chunk's first tile
};

// One token tile of the dW pass (LDS at xsb): recompute z, form dz = c1 * act'(z), accumulate
// db, dW and the tile's 4 mask bits (bit 4 (t % 8) + i of word mw for token i of tile t).  The
// first RA LDS reads of neuron j + 1 are issued before the arithmetic of neuron j.
// FM: the tile's mask bits come from the forward (fb: bit 15 - (4 j + i) = token i of neuron j): no z
// recompute, no W or bias; dz = c1 where the bit is set, else +0 (the bit sign-extended and ANDed
// with c1's pattern is the select below, bit for bit), and the bits go into mw as the recompute's.
template <int K, int NPL, int ACT, int RA, bool FAR, typename SRC = const char*, bool FM = false>
__device__ __forceinline__ void bwd_w_tile(SRC xsb, int t, const float4 c1, const unsigned (&addr)[NPL][K],
                                           const float (&w)[NPL][K], const float (&bias)[NPL], float (&dw)[NPL][K],
                                           float (&dbv)[NPL], unsigned (&mw)[NPL], unsigned fb) {
  float4 xc[K];
#pragma unroll
  for (int k = 0; k < RA; ++k) xc[k] = gather_x<FAR>(xsb, addr[0][k]);
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
#pragma unroll
    for (int k = RA; k < K; ++k) xc[k] = gather_x<FAR>(xsb, addr[j][k]);
    float4 xn[RA];
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xn[k] = gather_x<FAR>(xsb, addr[j + 1][k]);
    }
    __builtin_amdgcn_sched_barrier(0);
    float d0, d1, d2, d3;
    if constexpr (FM) {  // token i of neuron j is bit 15 - (4 j + i) of fb
      d0 = __uint_as_float((unsigned)__builtin_amdgcn_sbfe((int)fb, 15u - 4u * j, 1u) & __float_as_uint(c1.x));
      d1 = __uint_as_float((unsigned)__builtin_amdgcn_sbfe((int)fb, 14u - 4u * j, 1u) & __float_as_uint(c1.y));
      d2 = __uint_as_float((unsigned)__builtin_amdgcn_sbfe((int)fb, 13u - 4u * j, 1u) & __float_as_uint(c1.z));
      d3 = __uint_as_float((unsigned)__builtin_amdgcn_sbfe((int)fb, 12u - 4u * j, 1u) & __float_as_uint(c1.w));
      mw[j] |= ((unsigned)__builtin_bitreverse32(fb) >> (16u + 4u * j) & 15u) << ((t & 7) * 4);
    } else {
      float z0 = bias[j], z1 = bias[j], z2 = bias[j], z3 = bias[j];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        z0 = __builtin_fmaf(xc[k].x, w[j][k], z0);
        z1 = __builtin_fmaf(xc[k].y, w[j][k], z1);
        z2 = __builtin_fmaf(xc[k].z, w[j][k], z2);
        z3 = __builtin_fmaf(xc[k].w, w[j][k], z3);
      }
      const bool m0 = ACT != GL_ACT_RELU || z0 > 0.f, m1 = ACT != GL_ACT_RELU || z1 > 0.f;
      const bool m2 = ACT != GL_ACT_RELU || z2 > 0.f, m3 = ACT != GL_ACT_RELU || z3 > 0.f;
      d0 = m0 ? c1.x : 0.f, d1 = m1 ? c1.y : 0.f, d2 = m2 ? c1.z : 0.f, d3 = m3 ? c1.w : 0.f;
      mw[j] |= ((unsigned)m0 | ((unsigned)m1 << 1) | ((unsigned)m2 << 2) | ((unsigned)m3 << 3)) << ((t & 7) * 4);
    }
    dbv[j] = dbv[j] + d0 + d1 + d2 + d3;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      float a = dw[j][k];
      a = __builtin_fmaf(d0, xc[k].x, a);
      a = __builtin_fmaf(d1, xc[k].y, a);
      a = __builtin_fmaf(d2, xc[k].z, a);
      a = __builtin_fmaf(d3, xc[k].w, a);
      dw[j][k] = a;
    }
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xc[k] = xn[k];
    }
  }
}

// The same over a 4-token tile of raw bf16 values (8-byte slots): the gathers keep the packed
// words, which are widened (exactly) once after the read-ahead and used for both z and dW.
template <int K, int NPL, int ACT, int RA, bool FAR, bool FM = false>
__device__ __forceinline__ void bwd_w_tile_bf4(const char* xsb, int t, const float4 c1, const unsigned (&addr)[NPL][K],
                                               const float (&w)[NPL][K], const float (&bias)[NPL], float (&dw)[NPL][K],
                                               float (&dbv)[NPL], unsigned (&mw)[NPL], unsigned fb) {
  uint2 xr[K];
  auto ld = [&](unsigned a) {
    if constexpr (FAR) asm volatile("" : "+v"(a));
    return *reinterpret_cast<const uint2*>(xsb + a);
  };
#pragma unroll
  for (int k = 0; k < RA; ++k) xr[k] = ld(addr[0][k]);
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
#pragma unroll
    for (int k = RA; k < K; ++k) xr[k] = ld(addr[j][k]);
    uint2 xn[RA];
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xn[k] = ld(addr[j + 1][k]);
    }
    __builtin_amdgcn_sched_barrier(0);
    float4 xc[K];
#pragma unroll
    for (int k = 0; k < K; ++k)
      xc[k] = make_float4(__uint_as_float(xr[k].x << 16), __uint_as_float(xr[k].x & 0xffff0000u),
                          __uint_as_float(xr[k].y << 16), __uint_as_float(xr[k].y & 0xffff0000u));
    float d0, d1, d2, d3;
    if constexpr (FM) {  // token i of neuron j is bit 15 - (4 j + i) of fb
      d0 = __uint_as_float((unsigned)__builtin_amdgcn_sbfe((int)fb, 15u - 4u * j, 1u) & __float_as_uint(c1.x));
      d1 = __uint_as_float((unsigned)__builtin_amdgcn_sbfe((int)fb, 14u - 4u * j, 1u) & __float_as_uint(c1.y));
      d2 = __uint_as_float((unsigned)__builtin_amdgcn_sbfe((int)fb, 13u - 4u * j, 1u) & __float_as_uint(c1.z));
      d3 = __uint_as_float((unsigned)__builtin_amdgcn_sbfe((int)fb, 12u - 4u * j, 1u) & __float_as_uint(c1.w));
      mw[j] |= ((unsigned)__builtin_bitreverse32(fb) >> (16u + 4u * j) & 15u) << ((t & 7) * 4);
    } else {
      float z0 = bias[j], z1 = bias[j], z2 = bias[j], z3 = bias[j];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        z0 = __builtin_fmaf(xc[k].x, w[j][k], z0);
        z1 = __builtin_fmaf(xc[k].y, w[j][k], z1);
        z2 = __builtin_fmaf(xc[k].z, w[j][k], z2);
        z3 = __builtin_fmaf(xc[k].w, w[j][k], z3);
      }
      const bool m0 = ACT != GL_ACT_RELU || z0 > 0.f, m1 = ACT != GL_ACT_RELU || z1 > 0.f;
      const bool m2 = ACT != GL_ACT_RELU || z2 > 0.f, m3 = ACT != GL_ACT_RELU || z3 > 0.f;
      d0 = m0 ? c1.x : 0.f, d1 = m1 ? c1.y : 0.f, d2 = m2 ? c1.z : 0.f, d3 = m3 ? c1.w : 0.f;
      mw[j] |= ((unsigned)m0 | ((unsigned)m1 << 1) | ((unsigned)m2 << 2) | ((unsigned)m3 << 3)) << ((t & 7) * 4);
    }
    dbv[j] = dbv[j] + d0 + d1 + d2 + d3;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      float a = dw[j][k];
      a = __builtin_fmaf(d0, xc[k].x, a);
      a = __builtin_fmaf(d1, xc[k].y, a);
      a = __builtin_fmaf(d2, xc[k].z, a);
      a = __builtin_fmaf(d3, xc[k].w, a);
      dw[j][k] = a;
    }
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xr[k] = xn[k];
    }
  }
}

// The same over a two-token tile (8-byte slots): bits 2 (t % 16) + i of the mask word.
template <int K, int NPL, int ACT, int RA, bool FAR>
__device__ __forceinline__ void bwd_w_tile2(const char* xsb, int t, const float2 c1, const unsigned (&addr)[NPL][K],
                                            const float (&w)[NPL][K], const float (&bias)[NPL], float (&dw)[NPL][K],
                                            float (&dbv)[NPL], unsigned (&mw)[NPL]) {
  float2 xc[K];
#pragma unroll
  for (int k = 0; k < RA; ++k) xc[k] = gather_x2<FAR>(xsb, addr[0][k]);
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
#pragma unroll
    for (int k = RA; k < K; ++k) xc[k] = gather_x2<FAR>(xsb, addr[j][k]);
    float2 xn[RA];
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xn[k] = gather_x2<FAR>(xsb, addr[j + 1][k]);
    }
    __builtin_amdgcn_sched_barrier(0);
    float z0 = bias[j], z1 = bias[j];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      z0 = __builtin_fmaf(xc[k].x, w[j][k], z0);
      z1 = __builtin_fmaf(xc[k].y, w[j][k], z1);
    }
    const bool m0 = ACT != GL_ACT_RELU || z0 > 0.f, m1 = ACT != GL_ACT_RELU || z1 > 0.f;
    const float d0 = m0 ? c1.x : 0.f, d1 = m1 ? c1.y : 0.f;
    dbv[j] = dbv[j] + d0 + d1;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      float a = dw[j][k];
      a = __builtin_fmaf(d0, xc[k].x, a);
      a = __builtin_fmaf(d1, xc[k].y, a);
      dw[j][k] = a;
    }
    mw[j] |= ((unsigned)m0 | ((unsigned)m1 << 1)) << ((t & 15) * 2);
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xc[k] = xn[k];
    }
  }
}

// Token tiles reach LDS by LDS-DMA (dma_tile).  DBUF (D <= XTILE_DB): two buffers, tile t + 1
// lands while tile t is read; one tile body reads buffer (t & 1) through a run-time base, so the
// loop holds one copy of the gather code (two inlined copies, one per buffer, do not fit the 256
// VGPRs a wave has at 2 waves per SIMD with the dW accumulators live).  Otherwise one buffer:
// load, wait, read.  The wave index goes through readfirstlane so the chunk's parameters and the
// c1 row are addressed with scalar registers.
template <int K, int NPL, int WAVES, int ACT, int RA, bool DBUF, bool WS = false, bool XG = false, int TB = BT,
          bool XB = false, bool FM = false, bool SMALL = false>
__global__ void __launch_bounds__(WAVES * 64, SMALL ? 4 : 1) bwd_w_kernel(BwK p) {
  // XG (D > XTILE_SB): no LDS tile, the lanes gather from the token tiles in global memory.
  // TB: tokens per tile, 4 or 2 (two-token tiles in the two buffers of DBUF: D <= 2 XTILE_DB)
  static_assert(TB == BT || (TB == 2 && DBUF && !WS && !XG), "two-token tiles: double-buffered only");
  // XB: 4-token tiles of raw bf16 (8-byte slots, bf16 X), double- or small-buffered, or pool windows
  // staged from them
  static_assert(!XB || (TB == BT && (DBUF || SMALL || WS) && !XG), "bf16 tiles: double- or small-buffered, windows");
  // SMALL: one single-buffered 64-KiB tile per workgroup, two workgroups per CU (128 VGPRs at most)
  static_assert(!SMALL || (!DBUF && !WS && !XG && TB == BT), "small: one 4-token tile per workgroup");
  // FM: the mask bits come from the forward (p.fm): no z recompute, W and bias are not read
  static_assert(!FM || (TB == BT && ACT == GL_ACT_RELU), "forward ReLU bits: 4-token tiles, ReLU");
  constexpr unsigned SLOT = XB ? 8u : 4u * TB;  // bytes per input of a tile
  __shared__ float4 xs[DBUF || WS ? 2 * XTILE_DB : (XG ? 1 : (SMALL ? XTILE_DB : XTILE_SB))];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  long long chunk = (long long)blockIdx.x * WAVES + wave;
  const bool active = chunk < p.n_chunks;
  if (!active) chunk = p.n_chunks - 1;  // idle waves of the last block recompute a real chunk, store nothing
  const long long g = chunk / p.cpg;
  const int s_lo = (int)(chunk % p.cpg) * 64 * NPL;
  const int ext = pool_ext((int)g, p.S, p.sps, p.gs);  // slots of the pool inside its group
  const int n_g = min(p.counts[g], ext);

  unsigned addr[NPL][K];
  float w[NPL][K], dw[NPL][K];
  float bias[NPL], dbv[NPL];
  unsigned slot2[(NPL + 1) / 2];  // slots of neurons 2i, 2i+1 within the pool (16 bits each; >= n_g: padding)
  // window staging: this wave's pool is slot pk of the workgroup's staged pools, window start lo
  const int g_first = (int)((long long)blockIdx.x * WAVES / p.cpg);
  const int pk = WS ? (int)(g - g_first) : 0;
  const int lo = WS ? (int)__builtin_amdgcn_readfirstlane(p.win[g]) : 0;
  // the lane's neurons: LDS addresses of their inputs, weights, bias, slots
  if constexpr (WS) {
    // pool windows: the parameter dtype tested per load (the set-up below, written as a generic
    // lambda, raised these kernels' spills from 8 / 20 to 92 / 148 bytes per lane)
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      uint32_t order;
      const int s = sched_slot(p.sched, p.nwin, p.S, g, s_lo, j, lane, order);
      const unsigned s16 = (unsigned)(s < 0xffff ? s : 0xffff);
      if (j % 2 == 0) slot2[j / 2] = s16; else slot2[j / 2] |= s16 << 16;
      const bool valid = s < n_g;
      const long long n = pool_base((int)g, p.S, p.sps, p.gs) + (s < ext ? s : ext - 1);  // in bounds; invalid slots masked
#pragma unroll
      for (int ks = 0; ks < K; ++ks) {
        const int k = sched_k<K>(order, ks);
        int d = rec_index(p.idx, n, k, K, p.rs);
        d = (d < 0 || !valid) ? 0 : (d >= p.D ? p.D - 1 : d);  // host validates; clamp keeps LDS reads in bounds
        addr[j][ks] = win_addr<SLOT>(d, pk, lo, p.ww);
        if constexpr (!FM) {
          const float wl = ld_param(p.W, p.wbf, n * K + k);
          w[j][ks] = valid ? wl : 0.f;
        } else {
          w[j][ks] = 0.f;
        }
        dw[j][ks] = 0.f;
      }
      if constexpr (!FM) {
        const float bl = ld_param(p.bias, p.wbf, n);
        bias[j] = valid ? bl : 0.f;
      } else {
        bias[j] = 0.f;
      }
      dbv[j] = 0.f;
    }
  } else {
    // one uniform branch on the parameter dtype around the set-up, so the loads of either dtype
    // issue back to back (a dtype test per load made the compiler wait on each in turn)
    auto setup = [&](auto bf) {
      constexpr bool BF = decltype(bf)::value;
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        uint32_t order;
        const int s = sched_slot(p.sched, p.nwin, p.S, g, s_lo, j, lane, order);
        const unsigned s16 = (unsigned)(s < 0xffff ? s : 0xffff);
        if (j % 2 == 0) slot2[j / 2] = s16; else slot2[j / 2] |= s16 << 16;
        const bool valid = s < n_g;
        const long long n = pool_base((int)g, p.S, p.sps, p.gs) + (s < ext ? s : ext - 1);  // in bounds; invalid slots masked
#pragma unroll
        for (int ks = 0; ks < K; ++ks) {
          const int k = sched_k<K>(order, ks);
          int d = rec_index(p.idx, n, k, K, p.rs);
          d = (d < 0 || !valid) ? 0 : (d >= p.D ? p.D - 1 : d);  // host validates; clamp keeps LDS reads in bounds
          addr[j][ks] = (unsigned)d * SLOT;
          if constexpr (!FM) {
            const float wl = ld_param_t<BF>(p.W, n * K + k);
            w[j][ks] = valid ? wl : 0.f;
          } else {
            w[j][ks] = 0.f;
          }
          dw[j][ks] = 0.f;
        }
        if constexpr (!FM) {
          const float bl = ld_param_t<BF>(p.bias, n);
          bias[j] = valid ? bl : 0.f;
        } else {
          bias[j] = 0.f;
        }
        dbv[j] = 0.f;
      }
    };
    if (FM || !p.wbf) setup(std::false_type{});
    else setup(std::true_type{});
  }
  const float* c1row = p.c1t + g * p.cap;
  constexpr int NT = WAVES * 64;
  constexpr int TPW = 32 / TB;       // tiles per mask word
  const int ns = (int)((long long)p.D * SLOT / 16);  // 16-byte slots per tile (D even for 8-byte slots)

  // window staging: WS_TILES tiles per stage and barrier; tile t at slot (t mod 2 WS_TILES) * nsl
  const WinLayout L{p.win, p.ww, p.npw, g_first, p.G};
  const int nsl = p.npw * p.ww;
  const unsigned tstep = (unsigned)nsl * SLOT;
  const int rslots = WS_TILES * nsl * (int)SLOT / 16;  // 16-byte slots per stage region
  if constexpr (WS) {
    dma_window_stage<SLOT>(p.xt, xs, 0, p.n_tiles, p.D, L, WAVES);
    stage_wait();
    __syncthreads();
  } else if constexpr (DBUF) {
    dma_tile(p.xt, xs, ns, NT);
    stage_wait();
    __syncthreads();
  }
  // TPW token tiles (32 tokens) per mask word.  An even word is held in mwe until the odd word
  // after it is done, and the pair is stored as one 8-byte write: each store writes a separate
  // 32-byte memory sector, so pairs halve the mask's write traffic.
  unsigned mwe[NPL];
  // FM: the forward's 16 bits of this lane for tile t (coalesced 128 bytes per wave), loaded a tile ahead
  const uint16_t* fsrc = FM ? p.fm + (chunk * p.fm_tiles + p.fm_t0) * 64 + lane : nullptr;
  unsigned fbn = FM ? fsrc[0] : 0u;
  auto fbits = [&](int t) {
    const unsigned b = fbn;
    if (FM && t + 1 < p.n_tiles) fbn = fsrc[(long long)(t + 1) * 64];
    return b;
  };
  for (int t0 = 0; t0 < p.n_tiles; t0 += TPW) {
    unsigned mw[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) mw[j] = 0u;
    const int t1 = t0 + TPW < p.n_tiles ? t0 + TPW : p.n_tiles;
    if constexpr (WS) {
      for (int ts0 = t0; ts0 < t1; ts0 += WS_TILES) {
        const int r = (ts0 / WS_TILES) & 1;
        // region r ^ 1 was last read in the previous stage, which every wave finished before the barrier
        if (ts0 + WS_TILES < p.n_tiles)
          dma_window_stage<SLOT>(p.xt, xs + (r ^ 1) * rslots, ts0 + WS_TILES, p.n_tiles, p.D, L, WAVES);
        const int tn = p.n_tiles - ts0 < WS_TILES ? p.n_tiles - ts0 : WS_TILES;
        for (int tt = 0; tt < tn; ++tt) {
          const int t = ts0 + tt;
          const float4 c1 = ld_uniform4(c1row, t * BT);
          if constexpr (XB)
            bwd_w_tile_bf4<K, NPL, ACT, RA, false, FM>(reinterpret_cast<const char*>(xs), t, c1, addr, w, bias, dw, dbv,
                                                       mw, fbits(t));
          else
            bwd_w_tile<K, NPL, ACT, RA, false, const char*, FM>(reinterpret_cast<const char*>(xs), t, c1, addr, w, bias,
                                                               dw, dbv, mw, fbits(t));
          // next tile's slot; after the last tile of region 1 back to region 0 (uniform step, no branch)
          const unsigned step = (t & (2 * WS_TILES - 1)) == 2 * WS_TILES - 1 ? tstep - 2u * WS_TILES * tstep : tstep;
#pragma unroll
          for (int j = 0; j < NPL; ++j)
#pragma unroll
            for (int k = 0; k < K; ++k) addr[j][k] += step;
        }
        stage_wait();
        __syncthreads();
      }
    }
    for (int t = t0; t < t1 && !WS; ++t) {
      if constexpr (XG) {
        const float4 c1 = ld_uniform4(c1row, t * BT);
        bwd_w_tile<K, NPL, ACT, RA, false, decltype(xbuf(p.xt, p.D)), FM>(xbuf(p.xt + (long long)t * p.D, p.D), t, c1,
                                                                          addr, w, bias, dw, dbv, mw, fbits(t));
      } else if constexpr (DBUF) {
        // buffer cur ^ 1 was last read in tile t - 1, which every wave finished before the barrier
        const int cur = t & 1;
        if (t + 1 < p.n_tiles) dma_tile(p.xt + (long long)(t + 1) * ns, xs + (cur ^ 1) * XTILE_DB, ns, NT);
        if constexpr (XB) {
          const float4 c1 = ld_uniform4(c1row, t * BT);
          bwd_w_tile_bf4<K, NPL, ACT, RA, true, FM>(reinterpret_cast<const char*>(xs) + opaque(cur) * (XTILE_DB * 16),
                                                    t, c1, addr, w, bias, dw, dbv, mw, fbits(t));
        } else if constexpr (TB == 2) {
          const float2 c1 = ld_uniform2(c1row, t * 2);
          bwd_w_tile2<K, NPL, ACT, RA, true>(reinterpret_cast<const char*>(xs) + opaque(cur) * (XTILE_DB * 16), t, c1,
                                             addr, w, bias, dw, dbv, mw);
        } else {
          const float4 c1 = ld_uniform4(c1row, t * BT);
          bwd_w_tile<K, NPL, ACT, RA, true, const char*, FM>(
              reinterpret_cast<const char*>(xs) + opaque(cur) * (XTILE_DB * 16), t, c1, addr, w, bias, dw, dbv, mw,
              fbits(t));
        }
        stage_wait();  // tile t + 1 is in LDS for this wave's copies; the barrier publishes every wave's
        __syncthreads();
      } else {
        __syncthreads();  // every wave is done with tile t - 1
        dma_tile(p.xt + (long long)t * ns, xs, ns, NT);
        const float4 c1 = ld_uniform4(c1row, t * BT);
        stage_wait();
        __syncthreads();
        if constexpr (XB)
          bwd_w_tile_bf4<K, NPL, ACT, RA, false, FM>(reinterpret_cast<const char*>(xs), t, c1, addr, w, bias, dw, dbv,
                                                     mw, fbits(t));
        else
          bwd_w_tile<K, NPL, ACT, RA, false, const char*, FM>(reinterpret_cast<const char*>(xs), t, c1, addr, w, bias,
                                                             dw, dbv, mw, fbits(t));
      }
    }
    const int word = t0 / TPW;
    if ((word & 1) == 0 && t0 + TPW < p.n_tiles) {
#pragma unroll
      for (int j = 0; j < NPL; ++j) mwe[j] = mw[j];
      continue;
    }
    // odd word: (word - 1, word) in one row of one slab (mw2 is even); a last even word alone
    const int w0 = word & ~1;
    uint32_t* mslab = p.mask + ((long long)(w0 / p.mw2) * p.NS + pool_base((int)g, p.S, p.sps, p.gs)) * p.mw2 + w0 % p.mw2;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int s = (int)((opaque((int)slot2[j / 2]) >> (16 * (j % 2))) & 0xffff);  // address math kept local
      if (!active || s >= n_g) continue;
      if (word & 1)
        *reinterpret_cast<uint2*>(mslab + (long long)s * p.mw2) = make_uint2(mwe[j], mw[j]);
      else
        mslab[(long long)s * p.mw2] = mw[j];
    }
  }
  // mask words of tokens past the chunk are never written: their c1 is zero, so dX ignores them
  if (!active) return;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    uint32_t order;
    const int s = sched_slot(p.sched, p.nwin, p.S, g, s_lo, j, opaque(lane), order);
    if (s >= n_g) continue;
    const long long n = pool_base((int)g, p.S, p.sps, p.gs) + s;
#pragma unroll
    for (int ks = 0; ks < K; ++ks) p.dW[n * K + sched_k<K>(order, ks)] += dw[j][ks];
    p.db[n] += dbv[j];
  }
}

struct DxK {
  const uint32_t* __restrict__ rec;
  const uint32_t* __restrict__ seg_ptr;
  const int32_t* __restrict__ seg_unit;
  const uint32_t* __restrict__ seg_begin;
  const float* __restrict__ c1t;     // [G][cap]
  const uint32_t* __restrict__ mask;  // [n_tc][NS][2T]
  const float* __restrict__ W;
  float* part;  // [Q][D][cap]
  long long NS;
  int D, S, P, U, QL, UQ, FR, cap, n_tc;
  int sps, gs;  // pool geometry (pool_base)
  int wbf;      // W stored as bf16: the edge's weight is the half of the 32-bit word at (offset / 2) & ~3
  int ql0;      // dx_dense_kernel: the pass's first unit range per XCD (its ranges are ql0 .. ql0 + QL - 1)
};

// ---- dX ----------------------------------------------------------------------------------------
// One wave owns FW consecutive features, one range of UQ units and a slice of 64*T tokens: lane l
// holds tokens T*l .. T*l + T - 1 of the slice, whose activation bits are the T adjacent bits
// (T*l) % 32 .. of the neuron's mask word (T*l) / 32.  It walks the input-major edges of its
// features unit by unit, in the stored order, and for every edge (n, k) -> d adds
// c1[b, g(n)] * [mask[n, b]] * W[n, k] to the register accumulator of d.
//
// Edges are taken in chunks of up to 64 (one segment, or a 64-edge piece of a long one).  The
// lanes first gather, one edge each, the chunk's records, weights and mask words with vector
// loads (64 independent requests per instruction: random scalar loads would be limited by the
// scalar cache's miss rate); the gathers of the next chunk are issued before the current chunk is
// computed.  The chunk is staged in LDS as (mask word, weight) pairs, so for edge i every lane
// reads the word holding its bits and the weight with one ds_read_b64.  One v_bfe_u32 takes the
// lane's T bits, and a 2^T-entry LDS table turns them into T floats 0.0 / 1.0.
//
// A chunk belongs to one unit, so c1 is the same for all its edges: per run of edges into one
// feature the lanes sum S[j] = sum [mask] * W (one FMA per token and edge) and then add
// c1[j] * S[j] to the feature's accumulator (one FMA per token and run).
template <int T>
struct DxGather {
  unsigned rec;
  float w;
  unsigned m[2 * T];
};

struct DxChunk {
  int si;           // segment index
  unsigned e, end;  // chunk begin, segment end (edge positions)
  int u;            // unit of the segment
};

__device__ __forceinline__ void dx_next(const DxK& p, DxChunk& c, int hi) {
  if (c.e + 64 < c.end) {
    c.e += 64;
  } else {
    c.si += 1;
    if (c.si < hi) {
      c.e = c.end;
      c.end = p.seg_begin[c.si + 1];
      c.u = p.seg_unit[c.si];
    }
  }
}

// record of the lane's edge (lanes past the chunk take the chunk's first edge: in bounds, unused);
// the chunk's base address is wave-uniform (scalar registers), the lane adds a 32-bit offset
__device__ __forceinline__ unsigned dx_load_rec(const DxK& p, const DxChunk& c, int lane) {
  const unsigned n = min(c.end - c.e, 64u);
  return ld_uniform_u32(p.rec + c.e, (unsigned)lane < n ? (unsigned)lane * 4u : 0u);
}

template <int K, int T>
__device__ __forceinline__ void dx_gather(const DxK& p, const uint32_t* mask_tc, const DxChunk& c, unsigned rec,
                                          DxGather<T>& g) {
  const long long nb = pool_base(c.u / p.P, p.S, p.sps, p.gs) + (long long)(c.u % p.P) * US;  // first neuron of the unit
  const unsigned woff = rec & REC_OFF_MASK;  // byte offset of W[n, k] in the unit
  const unsigned nl = woff >> (K == 8 ? 5 : 6);
  g.rec = rec;
  // the unit's weight and mask rows start at wave-uniform addresses (scalar registers); each lane
  // adds a 32-bit offset (< 64 KiB), so the gathers need no 64-bit vector address arithmetic
  if (p.wbf) {
    const unsigned boff = woff >> 1;
    g.w = bf16_half(ld_uniform_u32(reinterpret_cast<const unsigned short*>(p.W) + nb * K, boff & ~3u), boff);
  } else {
    g.w = __uint_as_float(ld_uniform_u32(p.W + nb * K, woff));
  }
  const uint32_t* mb = mask_tc + nb * (2 * T);
  const unsigned mo = nl * (unsigned)(2 * T * 4);
  if constexpr (T == 1) {
    const uint2 v = ld_uniform_u64(mb, mo);
    g.m[0] = v.x, g.m[1] = v.y;
  } else {
#pragma unroll
    for (int h = 0; h < T / 2; ++h) {
      const uint4 v = ld_uniform_u128(mb, mo + 16u * h);
      g.m[4 * h] = v.x, g.m[4 * h + 1] = v.y, g.m[4 * h + 2] = v.z, g.m[4 * h + 3] = v.w;
    }
  }
}

// c1 of the lane's T tokens (tok0 = the first of them) for the pool of unit u
template <int T>
__device__ __forceinline__ void dx_load_c1(const DxK& p, int u, int tok0, float (&c1)[T]) {
  const float* c = p.c1t + (long long)(u / p.P) * p.cap + tok0;
  if constexpr (T == 4) {
    const float4 v = *reinterpret_cast<const float4*>(c);
    c1[0] = v.x, c1[1] = v.y, c1[2] = v.z, c1[3] = v.w;
  } else if constexpr (T == 2) {
    const float2 v = *reinterpret_cast<const float2*>(c);
    c1[0] = v.x, c1[1] = v.y;
  } else {
    c1[0] = c[0];
  }
}

// LDS copy of one chunk: per edge its 2T (mask word, weight) pairs, rows padded by one pair to
// 4T + 2 words (row e starts at bank 2 (2T + 1) e mod 64: the 32 lanes of each half of a 64-bit
// row write hit 32 different bank pairs); lut[v][j] = 1.0f when bit j of v is set, else 0.0f
template <int T>
struct __align__(16) DxStage {
  uint2 e[64][2 * T + 1];
  float lut[1 << T][T];
};

// the lane's T mask bits of word mw as floats 0.0 / 1.0
template <int T>
__device__ __forceinline__ void dx_bits(const DxStage<T>& st, unsigned mw, unsigned bit, float (&mf)[T]) {
  const unsigned v = __builtin_amdgcn_ubfe(mw, bit, (unsigned)T);
  if constexpr (T == 4) {
    const float4 t = *reinterpret_cast<const float4*>(&st.lut[v][0]);
    mf[0] = t.x, mf[1] = t.y, mf[2] = t.z, mf[3] = t.w;
  } else if constexpr (T == 2) {
    const float2 t = *reinterpret_cast<const float2*>(&st.lut[v][0]);
    mf[0] = t.x, mf[1] = t.y;
  } else {
    mf[0] = st.lut[v][0];
  }
}

// Edges i in [i0, i1) of the chunk, all into feature X of the range:
// acc[X][j] += c1[j] * sum_i [m_ij] w_i.
template <int X, int T>
__device__ __forceinline__ void dx_run(const DxStage<T>& st, int i0, int i1, int word, unsigned bit,
                                       const float (&c1)[T], float (&acc)[FW][T]) {
  // the run length as an opaque 32-bit scalar: compared on the scalar unit (bounds folded into the
  // 64-bit LDS address arithmetic were compared with 64-bit vector compares)
  int len = i1 - i0;
  asm volatile("" : "+s"(len));
  if (len <= 0) return;
  const uint2* e = &st.e[i0][word];
  float s[T], mf[T];
  uint2 mw = *e;
  dx_bits<T>(st, mw.x, bit, mf);
#pragma unroll
  for (int j = 0; j < T; ++j) s[j] = mf[j] * __uint_as_float(mw.y);
  for (int n = len - 1; n > 0; --n) {
    e += 2 * T + 1;
    mw = *e;
    dx_bits<T>(st, mw.x, bit, mf);
#pragma unroll
    for (int j = 0; j < T; ++j) s[j] = __builtin_fmaf(mf[j], __uint_as_float(mw.y), s[j]);
  }
#pragma unroll
  for (int j = 0; j < T; ++j) acc[X][j] = __builtin_fmaf(c1[j], s[j], acc[X][j]);
}

template <int X, int T>
__device__ __forceinline__ void dx_runs(const DxStage<T>& st, const int (&b)[FW + 1], int word, unsigned bit,
                                        const float (&c1)[T], float (&acc)[FW][T]) {
  dx_run<X, T>(st, b[X], b[X + 1], word, bit, c1, acc);
  if constexpr (X + 1 < FW) dx_runs<X + 1, T>(st, b, word, bit, c1, acc);
}

// The chunk's edges are sorted by feature: ballots give every feature's edge range, and one loop
// per feature (unrolled over the range) keeps every accumulator index a compile-time constant.
template <int T>
__device__ __forceinline__ void dx_compute(const DxGather<T>& g, DxStage<T>& st, int n, int lane, int word,
                                           unsigned bit, const float (&c1)[T], float (&acc)[FW][T]) {
  const unsigned wb = __float_as_uint(g.w);
#pragma unroll
  for (int i = 0; i < 2 * T; ++i) st.e[lane][i] = make_uint2(g.m[i], wb);
  __syncthreads();  // one wave per workgroup: orders the staging before the broadcast reads
  const int f = lane < n ? (int)((g.rec >> REC_F_SHIFT) & REC_F_MASK) : FW;
  int b[FW + 1];
  b[0] = 0;
#pragma unroll
  for (int x = 1; x <= FW; ++x)  // (readfirstlane keeps the bounds 32-bit: 64-bit compares are VALU)
    b[x] = __builtin_amdgcn_readfirstlane((int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(f < x)));
  dx_runs<0, T>(st, b, word, bit, c1, acc);
  __syncthreads();  // the next chunk's staging overwrites st
}

template <int K, int T>
__global__ void __launch_bounds__(64) dx_kernel(DxK p) {
  const int lane = threadIdx.x;
  // Workgroups are dispatched round-robin over the 8 XCDs.  All feature ranges of one unit range
  // run on the same XCD, side by side (F fastest), so the unit range's weights and mask words are
  // fetched into that XCD's L2 and shared by the waves of every feature range.
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int loc = bid >> 3;
  const int F = loc % p.FR;
  const int rest = loc / p.FR;
  const int ql = rest % p.QL;
  const int tc = rest / p.QL;
  const int q = ql * 8 + xcd;
  const int u_lo = q * p.UQ;
  const int u_hi = min(u_lo + p.UQ, p.U);
  int lo = (int)p.seg_ptr[F], hi = (int)p.seg_ptr[F + 1];
  {
    int a = lo, b = hi;
    while (a < b) {
      int mid = (a + b) >> 1;
      if (p.seg_unit[mid] < u_lo) a = mid + 1; else b = mid;
    }
    lo = a;
    b = hi;
    while (a < b) {
      int mid = (a + b) >> 1;
      if (p.seg_unit[mid] < u_hi) a = mid + 1; else b = mid;
    }
    hi = a;
  }
  float acc[FW][T];
#pragma unroll
  for (int f = 0; f < FW; ++f)
#pragma unroll
    for (int j = 0; j < T; ++j) acc[f][j] = 0.f;

  const int tok0 = tc * 64 * T + T * lane;
  const int word = (T * lane) >> 5;
  const unsigned bit = (unsigned)(T * lane) & 31u;
  const uint32_t* mask_tc = p.mask + (long long)tc * p.NS * (2 * T);
  __shared__ DxStage<T> st;
  if (lane < (1 << T)) {
#pragma unroll
    for (int j = 0; j < T; ++j) st.lut[lane][j] = (lane >> j) & 1 ? 1.0f : 0.0f;
  }
  if (lo < hi) {
    DxChunk cc{lo, p.seg_begin[lo], p.seg_begin[lo + 1], p.seg_unit[lo]};
    DxGather<T> gc;
    dx_gather<K, T>(p, mask_tc, cc, dx_load_rec(p, cc, lane), gc);
    float c1[T];
    dx_load_c1<T>(p, cc.u, tok0, c1);
    DxChunk cn = cc;
    dx_next(p, cn, hi);
    unsigned rn = cn.si < hi ? dx_load_rec(p, cn, lane) : 0u;
    for (;;) {
      // next chunk: gather (its records were requested one iteration ago), then request the
      // records of the chunk after it; both are in flight while the current chunk is computed
      const bool more = cn.si < hi;
      DxGather<T> gn = gc;
      float c1n[T];
#pragma unroll
      for (int j = 0; j < T; ++j) c1n[j] = c1[j];
      DxChunk cnn = cn;
      unsigned rnn = 0u;
      if (more) {
        dx_gather<K, T>(p, mask_tc, cn, rn, gn);
        if (cn.si != cc.si) dx_load_c1<T>(p, cn.u, tok0, c1n);
        dx_next(p, cnn, hi);
        if (cnn.si < hi) rnn = dx_load_rec(p, cnn, lane);
      }
      dx_compute<T>(gc, st, (int)min(cc.end - cc.e, 64u), lane, word, bit, c1, acc);
      if (!more) break;
      cc = cn;
      gc = gn;
#pragma unroll
      for (int j = 0; j < T; ++j) c1[j] = c1n[j];
      cn = cnn;
      rn = rnn;
    }
  }
  float* out = p.part + (long long)q * p.D * p.cap;
#pragma unroll
  for (int f = 0; f < FW; ++f) {
    const int d = F * FW + f;
    if (d < p.D) {
#pragma unroll
      for (int j = 0; j < T; ++j) out[(long long)d * p.cap + tok0 + j] = acc[f][j];
    }
  }
}

// The slice kernel (T = 4 tokens per lane and slice) with the chunk's gathers copied to LDS by the
// memory pipeline (global_load_lds): per edge the weight (one dword) and, for each of the wave's NS
// slices of 256 tokens, the neuron's 8 mask words of that slice (two 16-byte halves) land in a
// double buffer with no VGPR round trip and no staging stores.  NS = 1 holds 64 VGPRs (8 waves per
// SIMD); NS = 2 (512-token layers and up) walks each edge once for two slices, so the record, the
// weight, the run bounds and the per-chunk control are paid once per 512 tokens (4 waves per SIMD).
// The arithmetic of every token is dx_kernel's, in the same order.  LDS per wave: two buffers of
// [2 NS halves][64 edges] 16-byte mask quads and [64] weights, and the 16-entry bits-to-floats
// table.  A half holds 65 rows: row i of half h + 1 then sits 4 banks past row i of half h, so the
// two half-waves' reads of one edge (lanes 0-31 words 0-3, lanes 32-63 words 4-7) never share a bank.
template <int NS>
struct __align__(16) DxDma {
  uint4 m[2][2 * NS][65];
  float w[2][64];
  float lut[16][4];
};
// words between slice s and slice s + 1 of one half of a buffer
constexpr int DX_SLICE_WORDS = 2 * 65 * 4;

// the chunk's weights and the NS slices' mask rows -> buffer buf (lanes past the chunk copy the
// first edge's); slice s reads slab tc0 + s of the mask
template <int K, int NS>
__device__ __forceinline__ void dx_dma(const DxK& p, int tc0, const DxChunk& c, unsigned rec, DxDma<NS>& st, int buf) {
  const long long nb = pool_base(c.u / p.P, p.S, p.sps, p.gs) + (long long)(c.u % p.P) * US;  // first neuron of the unit
  const unsigned woff = rec & REC_OFF_MASK;  // byte offset of W[n, k] in the unit
  const unsigned mo = (woff >> (K == 8 ? 5 : 6)) * 32u;  // byte offset of the neuron's mask row
  // bf16 W: the 32-bit word holding the weight (its half is taken when the chunk is read)
  const unsigned wo = p.wbf ? (woff >> 1) & ~3u : woff;
  const char* ws = p.wbf ? uniform_ptr(reinterpret_cast<const unsigned short*>(p.W) + nb * K) : uniform_ptr(p.W + nb * K);
  const unsigned lw = __builtin_amdgcn_readfirstlane((unsigned)(size_t)&st.w[buf][0]);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, %2"
               :: "v"(wo), "s"(lw), "s"(ws) : "memory", "m0");
#pragma unroll
  for (int sl = 0; sl < NS; ++sl) {
    const char* ms = uniform_ptr(p.mask + ((long long)(tc0 + sl) * p.NS + nb) * 8);
    const unsigned l0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)&st.m[buf][2 * sl][0]);
    const unsigned l1 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)&st.m[buf][2 * sl + 1][0]);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %2"
                 :: "v"(mo), "s"(l0), "s"(ms) : "memory", "m0");
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %2"
                 :: "v"(mo + 16u), "s"(l1), "s"(ms) : "memory", "m0");
  }
}

// dx_run over the DMA layout: mrow = the lane's mask word of edge 0 in slice 0 (rows 16 bytes
// apart, slice s DX_SLICE_WORDS further); wl = the weight of the lane's own edge, edge i's weight
// taken from lane i (v_readlane, one VALU instead of one more LDS read per edge)
template <int X, int NS>
__device__ __forceinline__ void dx_run_dma(const unsigned* mrow, float wl, const float (*lut)[4], int i0, int i1,
                                           unsigned bit, const float (&c1)[NS][4], float (&acc)[NS][FW][4]) {
  int len = i1 - i0;
  asm volatile("" : "+s"(len));
  if (len <= 0) return;
  const unsigned* m = mrow + 4 * i0;
  float s[NS][4];
  {
    const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), i0));
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) {
      const unsigned v = __builtin_amdgcn_ubfe(m[sl * DX_SLICE_WORDS], bit, 4u);
      const float4 t = *reinterpret_cast<const float4*>(&lut[v][0]);
      s[sl][0] = t.x * wv, s[sl][1] = t.y * wv, s[sl][2] = t.z * wv, s[sl][3] = t.w * wv;
    }
  }
  for (int i = i0 + 1; i < i1; ++i) {
    m += 4;
    const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), i));
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) {
      const unsigned v = __builtin_amdgcn_ubfe(m[sl * DX_SLICE_WORDS], bit, 4u);
      const float4 t = *reinterpret_cast<const float4*>(&lut[v][0]);
      s[sl][0] = __builtin_fmaf(t.x, wv, s[sl][0]);
      s[sl][1] = __builtin_fmaf(t.y, wv, s[sl][1]);
      s[sl][2] = __builtin_fmaf(t.z, wv, s[sl][2]);
      s[sl][3] = __builtin_fmaf(t.w, wv, s[sl][3]);
    }
  }
#pragma unroll
  for (int sl = 0; sl < NS; ++sl)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[sl][X][j] = __builtin_fmaf(c1[sl][j], s[sl][j], acc[sl][X][j]);
}

template <int X, int NS>
__device__ __forceinline__ void dx_runs_dma(const unsigned* mrow, float wl, const float (*lut)[4],
                                            const int (&b)[FW + 1], unsigned bit, const float (&c1)[NS][4],
                                            float (&acc)[NS][FW][4]) {
  dx_run_dma<X, NS>(mrow, wl, lut, b[X], b[X + 1], bit, c1, acc);
  if constexpr (X + 1 < FW) dx_runs_dma<X + 1, NS>(mrow, wl, lut, b, bit, c1, acc);
}

// dx_next with the segment table read one step ahead: (pe, pu) hold the end and the unit of
// segment c.si + 1, loaded by the step that entered segment c.si; their loads land by the next
// loop-top wait, so no wait for them sits behind a chunk copy
__device__ __forceinline__ void dx_seg_ahead(const DxK& p, int si, int hi, unsigned& pe, unsigned& pu) {
  if (si + 1 < hi) {
    pe = p.seg_begin[si + 2];
    pu = (unsigned)p.seg_unit[si + 1];
  }
}
__device__ __forceinline__ void dx_next_ahead(const DxK& p, DxChunk& c, int hi, unsigned& pe, unsigned& pu) {
  if (c.e + 64 < c.end) {
    c.e += 64;
  } else {
    c.si += 1;
    if (c.si < hi) {
      c.e = c.end;
      c.end = __builtin_amdgcn_readfirstlane(pe);
      c.u = __builtin_amdgcn_readfirstlane((int)pu);
      dx_seg_ahead(p, c.si, hi, pe, pu);
    }
  }
}

// c1 of the lane's 4 tokens of each of the NS slices for the pool of unit u: a uniform row base
// (scalar registers) plus the lane's 32-bit offset (no 64-bit vector address to keep live)
template <int NS>
__device__ __forceinline__ void dx_load_c1_u(const DxK& p, int u, int slice0, int lane, float (&c1)[NS][4]) {
#pragma unroll
  for (int sl = 0; sl < NS; ++sl) {
    const uint4 v = ld_uniform_u128(p.c1t + (long long)(u / p.P) * p.cap + slice0 + sl * 256, (unsigned)lane * 16u);
    c1[sl][0] = __uint_as_float(v.x), c1[sl][1] = __uint_as_float(v.y), c1[sl][2] = __uint_as_float(v.z),
    c1[sl][3] = __uint_as_float(v.w);
  }
}

template <int K, int NS>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(NS == 1 ? 8 : 4, NS == 1 ? 8 : 4)))
dx_dma_kernel(DxK p) {
  constexpr int T = 4;
  const int lane = threadIdx.x;
  // block order as dx_kernel: all feature ranges of a unit range side by side on one XCD
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int loc = bid >> 3;
  const int F = loc % p.FR;
  const int rest = loc / p.FR;
  const int ql = rest % p.QL;
  const int tc0 = (rest / p.QL) * NS;  // the wave's first 256-token slice
  const int q = ql * 8 + xcd;
  const int u_lo = q * p.UQ;
  const int u_hi = min(u_lo + p.UQ, p.U);
  int lo = (int)p.seg_ptr[F], hi = (int)p.seg_ptr[F + 1];
  {
    int a = lo, b = hi;
    while (a < b) {
      int mid = (a + b) >> 1;
      if (p.seg_unit[mid] < u_lo) a = mid + 1; else b = mid;
    }
    lo = a;
    b = hi;
    while (a < b) {
      int mid = (a + b) >> 1;
      if (p.seg_unit[mid] < u_hi) a = mid + 1; else b = mid;
    }
    hi = a;
  }
  float acc[NS][FW][T];
#pragma unroll
  for (int sl = 0; sl < NS; ++sl)
#pragma unroll
    for (int f = 0; f < FW; ++f)
#pragma unroll
      for (int j = 0; j < T; ++j) acc[sl][f][j] = 0.f;

  const unsigned bit = (unsigned)(T * lane) & 31u;
  const int word = (T * lane) >> 5;  // the lane's word of a mask row: half word / 4, dword word % 4
  __shared__ DxDma<NS> st;
  if (lane < 16) {
#pragma unroll
    for (int j = 0; j < T; ++j) st.lut[lane][j] = (lane >> j) & 1 ? 1.0f : 0.0f;
  }
  if (lo < hi) {
    DxChunk cc{lo, p.seg_begin[lo], p.seg_begin[lo + 1], p.seg_unit[lo]};
    unsigned pe = 0u, pu = 0u;
    dx_seg_ahead(p, lo, hi, pe, pu);
    DxChunk cn = cc;
    dx_next_ahead(p, cn, hi, pe, pu);
    const unsigned rc0 = dx_load_rec(p, cc, lane);
    unsigned rn = cn.si < hi ? dx_load_rec(p, cn, lane) : 0u;
    dx_dma<K, NS>(p, tc0, cc, rc0, st, 0);
    unsigned rc = rc0;
    float c1[NS][T];
    dx_load_c1_u<NS>(p, cc.u, tc0 * 64 * T, lane, c1);
    int cur = 0;
    for (;;) {
      // every copy, load and LDS read so far is done: buffer cur holds chunk cc, and buffer
      // cur ^ 1 (read by the previous chunk) may be refilled
      __builtin_amdgcn_s_waitcnt(0);
      const bool more = cn.si < hi;
      float c1n[NS][T];
#pragma unroll
      for (int sl = 0; sl < NS; ++sl)
#pragma unroll
        for (int j = 0; j < T; ++j) c1n[sl][j] = c1[sl][j];
      DxChunk cnn = cn;
      unsigned rnn = 0u;
      if (more) {
        // the segment table before the copy: a wait for those loads after it would also wait for
        // the copy (the counter is in order); their values were loaded one step ago
        dx_next_ahead(p, cnn, hi, pe, pu);
        if (cnn.si < hi) rnn = dx_load_rec(p, cnn, lane);
        dx_dma<K, NS>(p, tc0, cn, rn, st, cur ^ 1);
        if (cn.si != cc.si) dx_load_c1_u<NS>(p, cn.u, tc0 * 64 * T, lane, c1n);
      }
      {
        const int n = (int)min(cc.end - cc.e, 64u);
        const int f = lane < n ? (int)((rc >> REC_F_SHIFT) & REC_F_MASK) : FW;
        int b[FW + 1];
        b[0] = 0;
#pragma unroll
        for (int x = 1; x <= FW; ++x)
          b[x] = __builtin_amdgcn_readfirstlane((int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(f < x)));
        const unsigned* mrow = reinterpret_cast<const unsigned*>(&st.m[opaque(cur)][word >> 2][0]) + (word & 3);
        float wl = st.w[opaque(cur)][lane];
        if (p.wbf) wl = bf16_half(__float_as_uint(wl), (rc & REC_OFF_MASK) >> 1);
        dx_runs_dma<0, NS>(mrow, wl, st.lut, b, bit, c1, acc);
      }
      if (!more) break;
      cc = cn;
      rc = rn;
#pragma unroll
      for (int sl = 0; sl < NS; ++sl)
#pragma unroll
        for (int j = 0; j < T; ++j) c1[sl][j] = c1n[sl][j];
      cn = cnn;
      rn = rnn;
      cur ^= 1;
    }
  }
  float* out = p.part + (long long)q * p.D * p.cap;
#pragma unroll
  for (int sl = 0; sl < NS; ++sl) {
    const int tok0 = (tc0 + sl) * 64 * T + T * lane;
#pragma unroll
    for (int f = 0; f < FW; ++f) {
      const int d = F * FW + f;
      if (d < p.D) {
#pragma unroll
        for (int j = 0; j < T; ++j) out[(long long)d * p.cap + tok0 + j] = acc[sl][f][j];
      }
    }
  }
}

// dX[b0 + b, d] = sum_q part[q, d, b]  (fixed order, q ascending), transposed to [B, D] through
// LDS.  A thread sums 4 adjacent tokens of one input with 16-byte loads, 8 partials in flight
// (the add order per element is unchanged); 32 inputs x 32 tokens per workgroup.  acc: the sum
// continues from the dX already there (the dense dX's later passes), so P passes over Q / P
// partials each add in the order of one pass over all Q.
__global__ void __launch_bounds__(256) dx_reduce_kernel(const float* __restrict__ part, float* __restrict__ dX, int D,
                                                        int cap, int Q, int b0, int Bc, int acc) {
  __shared__ float tile[32][33];  // [token][input]
  const int d0 = blockIdx.x * 32, bb = blockIdx.y * 32;
  const int dl = threadIdx.x >> 3, q4 = (threadIdx.x & 7) * 4;  // input d0 + dl, tokens bb + q4 .. + 3
  const int d = d0 + dl;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (acc) {  // the running sums, [B, D] rows in through the tile
    for (int r = threadIdx.x >> 5; r < 32; r += 8) {
      const int b = bb + r, dd = d0 + (threadIdx.x & 31);
      tile[r][threadIdx.x & 31] = dd < D && b < Bc ? dX[(long long)(b0 + b) * D + dd] : 0.f;
    }
    __syncthreads();
    v = make_float4(tile[q4][dl], tile[q4 + 1][dl], tile[q4 + 2][dl], tile[q4 + 3][dl]);
    __syncthreads();
  }
  if (d < D && bb + q4 < cap) {  // cap is a multiple of 64: the 4 tokens lie inside the partial rows
    const float4* src = reinterpret_cast<const float4*>(part + (long long)d * cap + bb + q4);
    const long long qs = (long long)D * cap / 4;  // float4 stride between partials
    int q = 0;
    for (; q + 8 <= Q; q += 8) {
      float4 t[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) t[i] = src[(q + i) * qs];
#pragma unroll
      for (int i = 0; i < 8; ++i) v.x += t[i].x, v.y += t[i].y, v.z += t[i].z, v.w += t[i].w;
    }
    for (; q < Q; ++q) {
      const float4 t = src[q * qs];
      v.x += t.x, v.y += t.y, v.z += t.z, v.w += t.w;
    }
  }
  tile[q4][dl] = v.x, tile[q4 + 1][dl] = v.y, tile[q4 + 2][dl] = v.z, tile[q4 + 3][dl] = v.w;
  __syncthreads();
  for (int r = threadIdx.x >> 5; r < 32; r += 8) {
    const int b = bb + r, dd = d0 + (threadIdx.x & 31);
    if (dd < D && b < Bc) dX[(long long)(b0 + b) * D + dd] = tile[r][threadIdx.x & 31];
  }
}

// ---- smooth pools (LogMeanExp, power mean, softmax-weighted) ------------------------------------
// Per (pool, token) coefficients (kernels/ops.py:242-262), transposed to [G][cap] like c1t:
//   sum / mean (GELU neurons): c1 = g_pre (/ n_g for mean)
//   LogMeanExp:       c1 = g_pre, c2 = L2 (from lse, or recovered as pre * scale + log2 n_g)
//   power mean:       c1 = g_pre / n_g, c2 = 1 / pre (both 0 when pre <= 0)
//   softmax-weighted: c1 = g_pre, c2 = L2, c3 = pre
// zero past the chunk's Bc tokens.
__global__ void __launch_bounds__(256) coef_smooth_kernel(const float* __restrict__ g_pre, const float* __restrict__ pre,
                                                          const float* __restrict__ lse, const int32_t* __restrict__ counts,
                                                          float* __restrict__ c1t, float* __restrict__ c2t,
                                                          float* __restrict__ c3t, int G, int b0, int Bc, int cap, int pool,
                                                          float scale) {
  __shared__ float tg[32][33], tp[32][33], tl[32][33];
  const int g0 = blockIdx.x * 32, bb = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int r = ty; r < 32; r += 8) {
    const int b = bb + r, g = g0 + tx;
    const bool in = b < Bc && g < G;
    const long long i = (long long)(b0 + b) * G + g;
    tg[r][tx] = in ? g_pre[i] : 0.f;
    tp[r][tx] = in && pre ? pre[i] : 0.f;
    tl[r][tx] = in && lse ? lse[i] : 0.f;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int g = g0 + r, b = bb + tx;
    if (g >= G || b >= cap) continue;
    const float gp = tg[tx][r], pv = tp[tx][r], L2 = tl[tx][r];
    const float n = (float)counts[g];
    float c1 = 0.f, c2 = 0.f, c3 = 0.f;
    if (b < Bc) {
      if (pool == GL_POOL_MEAN || pool == GL_POOL_SUM) {  // GELU neurons: c1t_kernel's c1
        c1 = pool == GL_POOL_MEAN ? gp / n : gp;
      } else if (pool == GL_POOL_POWER) {
        c1 = pv > 0.f ? gp / n : 0.f;
        c2 = pv > 0.f ? 1.f / pv : 0.f;
      } else {
        c1 = gp;
        c2 = lse ? L2 : pv * scale + __builtin_amdgcn_logf(n);
        c3 = pv;
      }
    }
    const long long o = (long long)g * cap + b;
    c1t[o] = c1, c2t[o] = c2, c3t[o] = c3;
  }
}

// dL/dz of one (token, neuron) of a smooth pool (triton_fused.py:364-399 _dz_from_z), or of sum /
// mean pooling with GELU (SM_LIN: c1 act'(z), triton_fused.py:364-374 for the mean coefficients)
template <int OP, int ACT>
__device__ __forceinline__ float smooth_dz(float z, float c1, float c2, float c3, float scale, float p, int pint) {
  if constexpr (OP == SM_LIN) {
    return c1 * dact_f<ACT>(z);
  } else if constexpr (OP == SM_POW) {
    if (!(z > 0.f)) return 0.f;
    const float q = z * c2;  // a / pre
    float qp;  // q^(p - 1)
    if (pint == 1) qp = 1.f;
    else if (pint == 2) qp = q;
    else if (pint == 4) qp = q * q * q;
    else if (pint == 8) { const float q2 = q * q, q4 = q2 * q2; qp = q4 * q2 * q; }
    else qp = q > 0.f ? __builtin_amdgcn_exp2f((p - 1.f) * __builtin_amdgcn_logf(q)) : 0.f;
    return c1 * qp;
  } else {
    const float a = act_f<ACT>(z);
    const float da = dact_f<ACT>(z);
    const float pw = __builtin_amdgcn_exp2f(a * scale - c2);
    if constexpr (OP == SM_SW) return c1 * pw * (1.f + p * (a - c3)) * da;
    return c1 * pw * da;
  }
}

struct BsK {
  const float4* __restrict__ xt;
  const int32_t* __restrict__ idx;
  const float* __restrict__ W;
  const float* __restrict__ bias;
  const int32_t* __restrict__ counts;
  const float* __restrict__ c1t;
  const float* __restrict__ c2t;
  const float* __restrict__ c3t;
  float* dW;
  float* db;
  float* dz;  // [G*S][cap] dL/dz of the chunk's tokens
  const uint32_t* sched;
  long long n_chunks;
  int D, S, cpg, n_tiles, cap, nwin, rs;
  float scale, pparam;
  int pint;
  int sps, gs;  // pool geometry (pool_base)
  int wbf;      // W and bias stored as bf16 (widened in the kernel)
};

// one step of a 4 x 4 transpose within a lane quad: lanes with b set give a, take the partner's c
template <int CTRL>
__device__ __forceinline__ void qswap(float4& a, float4& c, bool b) {
  // component-wise selects (a select of the two references would put the array in memory)
  const float s0 = b ? a.x : c.x, s1 = b ? a.y : c.y, s2 = b ? a.z : c.z, s3 = b ? a.w : c.w;
  const float r0 = dpp<CTRL>(s0), r1 = dpp<CTRL>(s1), r2 = dpp<CTRL>(s2), r3 = dpp<CTRL>(s3);
  a = make_float4(b ? r0 : a.x, b ? r1 : a.y, b ? r2 : a.z, b ? r3 : a.w);
  c = make_float4(b ? c.x : r0, b ? c.y : r1, b ? c.z : r2, b ? c.w : r3);
}

// Neuron-stationary recompute pass of a smooth pool: per token tile z, dz = c1 f(z, c2, c3), db and dW
// accumulated in registers over the chunk's tokens and added to the caller's buffers once; dz of
// every valid neuron stored for the dX pass.  Token tiles stream through LDS as in bwd_w_kernel.
template <int K, int NPL, int WAVES, int ACT, int OP, bool DBUF, bool XG = false, int SB = 1, int PI = -1>
__global__ void __launch_bounds__(WAVES * 64) bwd_smooth_kernel(BsK p) {
  // PI >= 0: the power mean's integer p (0: none) as a literal, so smooth_dz's powers fold
  const int pint = PI >= 0 ? PI : p.pint;
  // SB tiles of dz per neuron are held in registers and stored as one 16·SB-byte run: a lone
  // 16-byte piece of a row (rows are cap·4 bytes apart) is a partial line write
  static_assert(SB == 1 || SB == 2 || SB == 4 || SB == 8, "SB divides the 16 tiles of any cap");
  // XG (D > XTILE_SB): no LDS tile, the lanes gather from the token tiles in global memory
  __shared__ float4 xs[DBUF ? 2 * XTILE_DB : (XG ? 1 : XTILE_SB)];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  long long chunk = (long long)blockIdx.x * WAVES + wave;
  const bool active = chunk < p.n_chunks;
  if (!active) chunk = p.n_chunks - 1;
  const long long g = chunk / p.cpg;
  const int s_lo = (int)(chunk % p.cpg) * 64 * NPL;
  const int ext = pool_ext((int)g, p.S, p.sps, p.gs);  // slots of the pool inside its group
  const int n_g = min(p.counts[g], ext);
  const long long nb = pool_base((int)g, p.S, p.sps, p.gs);  // the pool's first neuron
  unsigned addr[NPL][K];
  float w[NPL][K], dw[NPL][K];
  float bias[NPL], dbv[NPL];
  int slot[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    uint32_t order;
    const int s = sched_slot(p.sched, p.nwin, p.S, g, s_lo, j, lane, order);
    slot[j] = s < n_g ? s : -1;
    const long long n = nb + (s < ext ? s : ext - 1);
#pragma unroll
    for (int ks = 0; ks < K; ++ks) {
      const int k = sched_k<K>(order, ks);
      int d = rec_index(p.idx, n, k, K, p.rs);
      d = (d < 0 || s >= n_g) ? 0 : (d >= p.D ? p.D - 1 : d);
      addr[j][ks] = (unsigned)d * 16u;
      w[j][ks] = s < n_g ? ld_param(p.W, p.wbf, n * K + k) : 0.f;
      dw[j][ks] = 0.f;
    }
    bias[j] = s < n_g ? ld_param(p.bias, p.wbf, n) : 0.f;
    dbv[j] = 0.f;
  }
  const float* c1row = p.c1t + g * p.cap;
  const float* c2row = p.c2t + g * p.cap;
  const float* c3row = p.c3t + g * p.cap;
  constexpr int NT = WAVES * 64;
  if constexpr (DBUF) {
    dma_tile(p.xt, xs, p.D, NT);
    stage_wait();
    __syncthreads();
  }
  float4 dzb[NPL][SB];
  for (int t0 = 0; t0 < p.n_tiles; t0 += SB) {
#pragma unroll
   for (int tt = 0; tt < SB; ++tt) {
    const int t = t0 + tt;
    if (t >= p.n_tiles) {  // past the last tile: zeros complete the run (cap is a multiple of 64 tokens)
#pragma unroll
      for (int j = 0; j < NPL; ++j) dzb[j][tt] = make_float4(0.f, 0.f, 0.f, 0.f);
      continue;
    }
    const char* xb = nullptr;
    const XBuf xg = xbuf(p.xt + (long long)t * p.D, p.D);  // XG: the tile in global memory
    if constexpr (XG) {
    } else if constexpr (DBUF) {
      const int cur = t & 1;
      if (t + 1 < p.n_tiles) dma_tile(p.xt + (long long)(t + 1) * p.D, xs + (cur ^ 1) * XTILE_DB, p.D, NT);
      xb = reinterpret_cast<const char*>(xs) + opaque(cur) * (XTILE_DB * 16);
    } else {
      __syncthreads();
      dma_tile(p.xt + (long long)t * p.D, xs, p.D, NT);
      stage_wait();
      __syncthreads();
      xb = reinterpret_cast<const char*>(xs);
    }
    const float4 c1 = ld_uniform4(c1row, t * BT), c2 = ld_uniform4(c2row, t * BT), c3 = ld_uniform4(c3row, t * BT);
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      float4 xc[K];
#pragma unroll
      for (int k = 0; k < K; ++k) xc[k] = XG ? gather_x<false>(xg, addr[j][k]) : gather_x<false>(xb, addr[j][k]);
      float z0 = bias[j], z1 = bias[j], z2 = bias[j], z3 = bias[j];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        z0 = __builtin_fmaf(xc[k].x, w[j][k], z0);
        z1 = __builtin_fmaf(xc[k].y, w[j][k], z1);
        z2 = __builtin_fmaf(xc[k].z, w[j][k], z2);
        z3 = __builtin_fmaf(xc[k].w, w[j][k], z3);
      }
      const bool v = slot[j] >= 0;
      const float d0 = v ? smooth_dz<OP, ACT>(z0, c1.x, c2.x, c3.x, p.scale, p.pparam, pint) : 0.f;
      const float d1 = v ? smooth_dz<OP, ACT>(z1, c1.y, c2.y, c3.y, p.scale, p.pparam, pint) : 0.f;
      const float d2 = v ? smooth_dz<OP, ACT>(z2, c1.z, c2.z, c3.z, p.scale, p.pparam, pint) : 0.f;
      const float d3 = v ? smooth_dz<OP, ACT>(z3, c1.w, c2.w, c3.w, p.scale, p.pparam, pint) : 0.f;
      dbv[j] = dbv[j] + d0 + d1 + d2 + d3;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        float a = dw[j][k];
        a = __builtin_fmaf(d0, xc[k].x, a);
        a = __builtin_fmaf(d1, xc[k].y, a);
        a = __builtin_fmaf(d2, xc[k].z, a);
        a = __builtin_fmaf(d3, xc[k].w, a);
        dw[j][k] = a;
      }
      dzb[j][tt] = make_float4(d0, d1, d2, d3);
    }
    if constexpr (DBUF) {
      stage_wait();
      __syncthreads();
    }
   }
    if constexpr (SB == 8) {
      // 4 x 4 transposes within each lane quad of pieces 0-3 and 4-7 of the runs: lane 4g + i ends
      // with piece 4h + i of neuron 4g + e's run in dzb[j][4h + e], so each store writes 64
      // contiguous bytes per quad where the lanes' own runs wrote 16 bytes per lane (a row apart):
      // C2 LogMeanExp recompute 36.2 -> 31.3 ms per 128-token chunk
      const bool q1 = lane & 1, q2 = lane & 2;
      const int qi = lane & 3;
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        qswap<0xB1>(dzb[j][0], dzb[j][1], q1);
        qswap<0xB1>(dzb[j][2], dzb[j][3], q1);
        qswap<0x4E>(dzb[j][0], dzb[j][2], q2);
        qswap<0x4E>(dzb[j][1], dzb[j][3], q2);
        qswap<0xB1>(dzb[j][4], dzb[j][5], q1);
        qswap<0xB1>(dzb[j][6], dzb[j][7], q1);
        qswap<0x4E>(dzb[j][4], dzb[j][6], q2);
        qswap<0x4E>(dzb[j][5], dzb[j][7], q2);
        // the slots of the quad's 4 neurons (quad_perm broadcasts; -1: past the pool)
        const int s0 = __builtin_amdgcn_update_dpp(0, slot[j], 0x00, 0xf, 0xf, false);
        const int s1 = __builtin_amdgcn_update_dpp(0, slot[j], 0x55, 0xf, 0xf, false);
        const int s2 = __builtin_amdgcn_update_dpp(0, slot[j], 0xAA, 0xf, 0xf, false);
        const int s3 = __builtin_amdgcn_update_dpp(0, slot[j], 0xFF, 0xf, 0xf, false);
        if (active && s0 >= 0) {
          float4* dst = reinterpret_cast<float4*>(p.dz + (nb + s0) * (long long)p.cap + t0 * BT);
          dst[qi] = dzb[j][0], dst[4 + qi] = dzb[j][4];
        }
        if (active && s1 >= 0) {
          float4* dst = reinterpret_cast<float4*>(p.dz + (nb + s1) * (long long)p.cap + t0 * BT);
          dst[qi] = dzb[j][1], dst[4 + qi] = dzb[j][5];
        }
        if (active && s2 >= 0) {
          float4* dst = reinterpret_cast<float4*>(p.dz + (nb + s2) * (long long)p.cap + t0 * BT);
          dst[qi] = dzb[j][2], dst[4 + qi] = dzb[j][6];
        }
        if (active && s3 >= 0) {
          float4* dst = reinterpret_cast<float4*>(p.dz + (nb + s3) * (long long)p.cap + t0 * BT);
          dst[qi] = dzb[j][3], dst[4 + qi] = dzb[j][7];
        }
      }
    } else if constexpr (SB == 2) {
      // fan-in 16 (2-tile runs): a 2 x 2 transpose within each lane pair, so each store writes 32
      // contiguous bytes per pair (C5-shape LogMeanExp recompute 66.1 -> 60.8 ms per 256-token chunk)
      const bool q1 = lane & 1;
      const int qi = lane & 1;
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        qswap<0xB1>(dzb[j][0], dzb[j][1], q1);
        const int s0 = __builtin_amdgcn_update_dpp(0, slot[j], 0xA0, 0xf, 0xf, false);  // quad_perm(0,0,2,2)
        const int s1 = __builtin_amdgcn_update_dpp(0, slot[j], 0xF5, 0xf, 0xf, false);  // quad_perm(1,1,3,3)
        if (active && s0 >= 0) reinterpret_cast<float4*>(p.dz + (nb + s0) * (long long)p.cap + t0 * BT)[qi] = dzb[j][0];
        if (active && s1 >= 0) reinterpret_cast<float4*>(p.dz + (nb + s1) * (long long)p.cap + t0 * BT)[qi] = dzb[j][1];
      }
    } else {
#pragma unroll
      for (int j = 0; j < NPL; ++j)
        if (active && slot[j] >= 0) {
          float4* dst = reinterpret_cast<float4*>(p.dz + (nb + slot[j]) * (long long)p.cap + t0 * BT);
#pragma unroll
          for (int tt = 0; tt < SB; ++tt) dst[tt] = dzb[j][tt];
        }
    }
  }
  if (!active) return;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    uint32_t order;
    const int s = sched_slot(p.sched, p.nwin, p.S, g, s_lo, j, opaque(lane), order);
    if (s >= n_g) continue;
    const long long n = pool_base((int)g, p.S, p.sps, p.gs) + s;
#pragma unroll
    for (int ks = 0; ks < K; ++ks) p.dW[n * K + sched_k<K>(order, ks)] += dw[j][ks];
    p.db[n] += dbv[j];
  }
}

// dX of a smooth pool: dX[b, d] = sum over edges (n, k) -> d of dz[b, n] W[n, k], walking the
// input-major edges like dx_kernel (one wave per feature range, unit range and token slice); per
// edge every lane reads its T tokens of the neuron's dz row (T = 1, 2 or 4 for token chunks of up
// to 64, 128 or 256 tokens; test_gpu_smooth's B = 130 case runs T = 4).  A segment's edges are sorted
// by feature, so consecutive edges into one feature are summed in registers (a run) and the run is
// added to that feature's sums in LDS when the feature changes: one uniform branch per run where
// selecting one of FW register accumulators per edge cost FW * T multiply-adds and selects.
template <int K, int T>
__global__ void __launch_bounds__(64) dx_dense_kernel(DxK p, const float* __restrict__ dz) {
  const int lane = threadIdx.x;
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int loc = bid >> 3;
  const int F = loc % p.FR;
  const int rest = loc / p.FR;
  const int ql = rest % p.QL;
  const int tc = rest / p.QL;
  const int q = ql * 8 + xcd;                        // the pass's partial slot
  const int u_lo = ((p.ql0 + ql) * 8 + xcd) * p.UQ;  // the layer's unit range (p.ql0 + ql) * 8 + xcd
  const int u_hi = min(u_lo + p.UQ, p.U);
  int lo = (int)p.seg_ptr[F], hi = (int)p.seg_ptr[F + 1];
  {
    int a = lo, b = hi;
    while (a < b) {
      int mid = (a + b) >> 1;
      if (p.seg_unit[mid] < u_lo) a = mid + 1; else b = mid;
    }
    lo = a;
    b = hi;
    while (a < b) {
      int mid = (a + b) >> 1;
      if (p.seg_unit[mid] < u_hi) a = mid + 1; else b = mid;
    }
    hi = a;
  }
  const int tok0 = tc * 64 * T + T * lane;
  __shared__ uint2 st[64];  // (record, weight bits) of the chunk's edges
  // per feature of the range, every lane's T sums: lane-major rows of T floats (no bank conflicts)
  __shared__ float sums[FW][64 * T];
#pragma unroll
  for (int x = 0; x < FW; ++x)
#pragma unroll
    for (int j = 0; j < T; ++j) sums[x][T * lane + j] = 0.f;
  float r[T];  // the open run: its feature fc (wave-uniform; -1 before the first edge)
#pragma unroll
  for (int j = 0; j < T; ++j) r[j] = 0.f;
  int fc = -1;
  const unsigned lo8 = (unsigned)tok0 * 4u;  // the lane's byte offset in a dz row
  for (int si = lo; si < hi; ++si) {
    const int u = p.seg_unit[si];
    const long long nb = pool_base(u / p.P, p.S, p.sps, p.gs) + (long long)(u % p.P) * US;  // first neuron of the unit
    const unsigned e_end = p.seg_begin[si + 1];
    for (unsigned e0 = p.seg_begin[si]; e0 < e_end; e0 += 64) {
      const int n = (int)min(e_end - e0, 64u);
      if (lane < n) {
        const unsigned rec = p.rec[e0 + lane];
        const float wv = ld_param(p.W, p.wbf, nb * K + (long long)((rec & REC_OFF_MASK) >> 2));
        st[lane] = make_uint2(rec, __float_as_uint(wv));
      }
      __syncthreads();
      // DB edges at a time: their dz rows are loaded together (DB loads in flight per wave, where
      // one dependent load per edge exposed each load's latency), then added in edge order.  With
      // the unit-range passes most rows come from the caches, and fewer rows in flight (fewer
      // VGPRs, more waves) pay: at 2 tokens per lane (C2, 128-token chunks) 3.63 / 3.37 / 3.24 /
      // 3.40 ms per pass for DB = 8 / 4 / 3 / 2; at 4 tokens per lane (C5 shape) DB = 4 3.58 ms, 2 3.99
      constexpr int DB = T == 4 ? 4 : (T == 2 ? 3 : 8);
      for (int i0 = 0; i0 < n; i0 += DB) {
        float v[DB][T], wv[DB];
        int f[DB];
#pragma unroll
        for (int u = 0; u < DB; ++u) {
          const int i = i0 + u < n ? i0 + u : n - 1;  // past the chunk: the last edge again, not added
          uint2 e = st[i];
          e.x = __builtin_amdgcn_readfirstlane(e.x);  // the same edge in every lane
          e.y = __builtin_amdgcn_readfirstlane(e.y);
          f[u] = i0 + u < n ? (int)((e.x >> REC_F_SHIFT) & REC_F_MASK) : FW;
          const long long nn = nb + ((e.x & REC_OFF_MASK) >> (K == 8 ? 5 : 6));
          wv[u] = __uint_as_float(e.y);
          const float* row = dz + nn * p.cap;  // scalar row base (buffer resource), the lane's 32-bit offset
          if constexpr (T == 4) {
            const uint4 x = ld_uniform_u128(row, lo8);
            v[u][0] = __uint_as_float(x.x), v[u][1] = __uint_as_float(x.y);
            v[u][2] = __uint_as_float(x.z), v[u][3] = __uint_as_float(x.w);
          } else if constexpr (T == 2) {
            const uint2 x = ld_uniform_u64(row, lo8);
            v[u][0] = __uint_as_float(x.x), v[u][1] = __uint_as_float(x.y);
          } else {
            v[u][0] = __uint_as_float(ld_uniform_u32(row, lo8));
          }
        }
#pragma unroll
        for (int u = 0; u < DB; ++u) {
          if (f[u] >= FW) break;  // past the chunk (uniform)
          if (f[u] != fc) {       // the run ends: add it to its feature's sums
            if (fc >= 0) {
#pragma unroll
              for (int j = 0; j < T; ++j) sums[fc][T * lane + j] += r[j];
            }
            fc = f[u];
#pragma unroll
            for (int j = 0; j < T; ++j) r[j] = 0.f;
          }
#pragma unroll
          for (int j = 0; j < T; ++j) r[j] = __builtin_fmaf(wv[u], v[u][j], r[j]);
        }
      }
      __syncthreads();
    }
  }
  if (fc >= 0) {
#pragma unroll
    for (int j = 0; j < T; ++j) sums[fc][T * lane + j] += r[j];
  }
  float* out = p.part + (long long)q * p.D * p.cap;
#pragma unroll
  for (int x = 0; x < FW; ++x) {
    const int d = F * FW + x;
    if (d < p.D) {
#pragma unroll
      for (int j = 0; j < T; ++j) out[(long long)d * p.cap + tok0 + j] = sums[x][T * lane + j];
    }
  }
}

// ---- host side -------------------------------------------------------------------------------
// dW pass: 4 neurons per lane in 12 waves at K = 8 (3 waves per SIMD, 3072 neurons per staged
// token tile), 2 in 8 waves at K = 16 (2 waves per SIMD at ~188 VGPRs, 1024 neurons per tile):
// chunks of 128 slots cover pools of 512 exactly, where 3 per lane (chunks of 192) left 11% of the
// lanes idle (C5 dW 53.8 -> 52.8 ms)
constexpr int bwd_npl(int K) { return K == 8 ? 4 : 2; }
static_assert(bwd_npl(8) == RELU_MASK_NPL, "the dW pass reads the forward's ReLU bits chunk by chunk");
// The smooth pools' recompute pass keeps every gathered x of a neuron live across dz, and holds
// smooth_sb tiles of dz per neuron to store them as one 128-byte (K = 8) or 32-byte (K = 16) run:
// 2 neurons per lane.  At K = 8, 4 per lane with 16-byte stores ran 28.5 ms per 64-token C2
// chunk, 2 per lane with 64-byte runs 22.0 ms, with 128-byte runs 22.6 ms (4 per lane with 32-byte
// runs spills); per 128-token chunk (the layer's default dz budget) 64-byte runs 37.6 ms,
// 128-byte runs 35.5 ms.
constexpr int smooth_npl(int K) { return 2; }
constexpr int smooth_sb(int K) { return K == 8 ? 8 : 2; }
constexpr int bwd_waves(int K) { return K == 8 ? 12 : 8; }
#ifndef DX_DMA_TWO_SLICES
#define DX_DMA_TWO_SLICES 1
#endif
#ifndef BWD_FM_WAVES
#define BWD_FM_WAVES 16
#endif
#ifndef BWD_FM_SMALL
#define BWD_FM_SMALL 1
#endif
#ifndef BWD_FM_RA
#define BWD_FM_RA 1
#endif
// kept bits with pool windows: waves per workgroup and read-ahead (12 waves: 132 VGPRs, where 16
// waves held to 128 spilled 20 bytes per lane; C3 dW 19.6 -> 18.9 ms)
#ifndef BWD_FM_WIN_WAVES
#define BWD_FM_WIN_WAVES 12
#endif
#ifndef BWD_FM_WIN_RA
#define BWD_FM_WIN_RA 1
#endif

struct BwdPlan {
  int bc_max, npl, waves, cpg, tiles_max, cap_max, rs_max, FR, P, U, Q, QL, UQ;
  int QLs, UQs;  // the dense dX: unit ranges per XCD and units per range (passes of QL ranges)
  long long n_chunks, e_max, nseg_max;
  size_t xt_bytes, c1_bytes, mask_bytes, part_bytes, edges_bytes, dz_bytes;
};

// smooth pools keep dz [G*S][cap] of one token chunk: chunks of at most 1024 tokens whose dz fits
// the caller's dz_budget, or SMOOTH_DZ_BUDGET (at least 64 tokens).  Larger chunks cost less per
// token: at C2, 64-token chunks ran 0.34 + 0.90 ms per token (recompute + dX), 128-token chunks
// 0.29 + 0.60, 256-token chunks 0.33 + 0.52
constexpr size_t SMOOTH_DZ_BUDGET = 8ull << 30;
static bool is_smooth(int pool) { return pool == GL_POOL_LME || pool == GL_POOL_POWER || pool == GL_POOL_SOFTMAX; }
// backward through a per-neuron dz (recompute pass + dense dX): the smooth pools, and sum / mean
// pooling of GELU neurons (dz = c1 gelu'(z) is not a 0 / 1 mask times c1)
static bool dense_dz(int pool, int act) {
  return is_smooth(pool) || (act == GL_ACT_GELU && (pool == GL_POOL_MEAN || pool == GL_POOL_SUM));
}

static BwdPlan bwd_plan(int B, int D, int G, int S, int K, bool smooth = false, size_t dz_budget = 0) {
  BwdPlan q;
  q.bc_max = B < BWD_TOKEN_CHUNK ? B : BWD_TOKEN_CHUNK;
  if (smooth) {
    long long c = (long long)((dz_budget ? dz_budget : SMOOTH_DZ_BUDGET) / ((size_t)G * S * 4)) / 64 * 64;
    if (c < 64) c = 64;
    if (c < q.bc_max) q.bc_max = (int)c;
  }
  q.npl = smooth ? smooth_npl(K) : bwd_npl(K);
  q.waves = bwd_waves(K);
  q.cpg = ceil_div(S, 64 * q.npl);
  q.n_chunks = (long long)G * q.cpg;
  q.tiles_max = ceil_div(q.bc_max, BT);
  q.cap_max = dx_cap(q.bc_max);
  q.rs_max = mask_stride(q.bc_max);
  q.FR = ceil_div(D, FW);
  q.P = ceil_div(S, US);
  q.U = G * q.P;
  // Q = 8 * QL unit ranges (one set of QL per XCD).  Short ranges keep the feature-range waves
  // that share a unit close together in time, so the unit's weights and mask words are still in
  // the XCD's L2 when the next of them gathers from it (measured at C2: QL 8 -> 32 cut the dX
  // kernel by 8% for 0.3 ms more partial-sum reduction).  About 256K waves in total, at most
  // QL = 32 and at least 128 units per range, so the [Q, D, tokens] partials (and their
  // reduction) stay small next to the layer -- except that small layers get shorter ranges until
  // they have 16K waves (two per wave slot of the chip): at C1 (4096 units) 4 ranges per XCD left
  // 4096 waves walking 128 units each, a latency-bound 0.29 ms against 0.20 ms with 16.
  const int n_tc = q.cap_max / (64 * dx_slots(q.bc_max));
  const long long waves_wanted = 262144;
  long long ql = (waves_wanted + 8LL * q.FR * n_tc - 1) / (8LL * q.FR * n_tc);
  if (ql > 32) ql = 32;
  const long long ql_fill = (16384 + 8LL * q.FR * n_tc - 1) / (8LL * q.FR * n_tc);
  if (ql > q.U / 1024 && ql > ql_fill) ql = q.U / 1024 > ql_fill ? q.U / 1024 : ql_fill;
  if (ql < 1) ql = 1;
  if (8 * ql > q.U) ql = ceil_div(q.U, 8);
  q.QL = (int)ql;
  q.Q = 8 * q.QL;
  q.UQ = ceil_div(q.U, q.Q);
  // The dense dX (per-neuron dz) reads a neuron's 4·cap-byte dz row once per edge, and mostly
  // from HBM unless the feature-range waves that share a unit read it close together in time.
  // Short unit ranges keep them together: ranges of ~192 KiB of dz rows per wave,
  // Q = E · 256 T / (FR · 192 KiB) (at C2 LogMeanExp, 128-token chunks: ranges of 24 units,
  // dX 67.6 -> 57.0 ms per chunk; 12 units 59.4, 48 units 58.4; at the C5 shape 256-token chunks
  // 189.5 -> 113.6 ms with ranges of 12 units, 133.3 with 24).  The ranges run as passes of QL
  // ranges per XCD into the same [Q][D][cap] partials, each reduced onto the last.
  q.QLs = q.QL;
  q.UQs = q.UQ;
  if (smooth) {
    const long long tb = 256LL * dx_slots(q.bc_max);  // dz bytes per edge and 64-lane wave
    long long qls = (long long)G * S * K * tb / ((long long)q.FR * (192 << 10)) / 8;
    if (qls > 2048) qls = 2048;
    if (qls > q.U / 8) qls = q.U / 8;  // at least one unit per range
    if (qls >= 2 * q.QL) {
      q.QLs = (int)(qls / q.QL * q.QL);
      q.UQs = ceil_div(q.U, 8 * q.QLs);
    }
  }
  q.xt_bytes = (size_t)round_up((long long)q.tiles_max * D * 16, 256);
  q.c1_bytes = (size_t)round_up((long long)G * q.cap_max * 4, 256);
  q.mask_bytes = (size_t)round_up((long long)G * S * q.rs_max * 4, 256);
  q.dz_bytes = smooth ? (size_t)round_up((long long)G * S * q.cap_max * 4, 256) : 0;
  if (smooth) q.mask_bytes = 0;
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

template <int K, int NPL, int WAVES, int ACT, int RA>
static int launch_bwd_w(const BwK& k, hipStream_t s) {
  auto fn = k.win ? (k.xb ? bwd_w_kernel<K, NPL, WAVES, ACT, RA, false, true, false, BT, true>
                          : bwd_w_kernel<K, NPL, WAVES, ACT, RA, false, true>)
                  : k.xb ? bwd_w_kernel<K, NPL, WAVES, ACT, RA, true, false, false, BT, true>
                  : k.tb == 2 ? bwd_w_kernel<K, NPL, WAVES, ACT, RA, true, false, false, 2>
                  : (k.D <= XTILE_DB ? bwd_w_kernel<K, NPL, WAVES, ACT, RA, true>
                                     : (k.D <= XTILE_SB ? bwd_w_kernel<K, NPL, WAVES, ACT, RA, false>
                                                        : bwd_w_kernel<K, NPL, WAVES, ACT, RA, false, false, true>));

  GL_LAUNCH(k.win ? GL_KERNEL_BWD_W_WIN : GL_KERNEL_BWD_W, fn, dim3((unsigned)ceil_div(k.n_chunks, WAVES)),
            dim3(WAVES * 64), 0, s, k);
  GL_CHECK_LAUNCH();
  return 0;
}

// With the forward's ReLU bits (gl_bwd checked the format) the dW pass holds neither W nor bias
// and fits 128 VGPRs: 16 waves per workgroup, 4 per SIMD.
template <int K, int NPL, int WAVES, int RA>
static int launch_bwd_w_fm(const BwK& k, hipStream_t s) {
  constexpr int A = GL_ACT_RELU;
  // full tiles of at most 64 KiB (fp32 D <= 4096, bf16 D <= 8192): two workgroups of WAVES / 2
  // waves per CU, each with one single-buffered tile, the forward's arrangement: while one waits
  // at its tile barrier the other computes
  if (BWD_FM_SMALL && !k.win && (k.xb || k.D <= XTILE_DB)) {
    constexpr int W2 = WAVES / 2;
    auto fs = k.xb ? bwd_w_kernel<K, NPL, W2, A, RA, false, false, false, BT, true, true, true>
                   : bwd_w_kernel<K, NPL, W2, A, RA, false, false, false, BT, false, true, true>;
    GL_LAUNCH(GL_KERNEL_BWD_W, fs, dim3((unsigned)ceil_div(k.n_chunks, W2)), dim3(W2 * 64), 0, s, k);
    GL_CHECK_LAUNCH();
    return 0;
  }
  if (k.win) {
    constexpr int WW = BWD_FM_WIN_WAVES;
    auto fw = k.xb ? bwd_w_kernel<K, NPL, WW, A, BWD_FM_WIN_RA, false, true, false, BT, true, true>
                   : bwd_w_kernel<K, NPL, WW, A, BWD_FM_WIN_RA, false, true, false, BT, false, true>;
    GL_LAUNCH(GL_KERNEL_BWD_W_WIN, fw, dim3((unsigned)ceil_div(k.n_chunks, WW)), dim3(WW * 64), 0, s, k);
    GL_CHECK_LAUNCH();
    return 0;
  }
  auto fn = k.xb ? bwd_w_kernel<K, NPL, WAVES, A, RA, true, false, false, BT, true, true>
            : (k.D <= XTILE_DB ? bwd_w_kernel<K, NPL, WAVES, A, RA, true, false, false, BT, false, true>
                               : (k.D <= XTILE_SB ? bwd_w_kernel<K, NPL, WAVES, A, RA, false, false, false, BT, false, true>
                                                  : bwd_w_kernel<K, NPL, WAVES, A, RA, false, false, true, BT, false, true>));
  GL_LAUNCH(GL_KERNEL_BWD_W, fn, dim3((unsigned)ceil_div(k.n_chunks, WAVES)), dim3(WAVES * 64), 0, s, k);
  GL_CHECK_LAUNCH();
  return 0;
}

// read-ahead of 2 LDS reads (more would spill)
template <int ACT>
static int launch_bwd_w_act(int K, const BwK& k, hipStream_t s) {
  if constexpr (ACT == GL_ACT_RELU)
    if (K == 8 && k.fm) return launch_bwd_w_fm<8, bwd_npl(8), BWD_FM_WAVES, BWD_FM_RA>(k, s);
  if (K == 8) return launch_bwd_w<8, bwd_npl(8), bwd_waves(8), ACT, 2>(k, s);
  return launch_bwd_w<16, bwd_npl(16), bwd_waves(16), ACT, 2>(k, s);
}

static int launch_bwd_w_any(int K, int act, const BwK& k, hipStream_t s) {
  return act == GL_ACT_RELU ? launch_bwd_w_act<GL_ACT_RELU>(K, k, s) : launch_bwd_w_act<GL_ACT_IDENTITY>(K, k, s);
}

template <int K, int T>
static int launch_dx_kt(const DxK& k, hipStream_t s, bool dma) {
  if constexpr (T == 4) {
    if (dma) {  // two 256-token slices per wave when the chunk has an even number of them
      const bool two = k.n_tc % 2 == 0 && DX_DMA_TWO_SLICES;
      auto fn = two ? dx_dma_kernel<K, 2> : dx_dma_kernel<K, 1>;
      GL_LAUNCH(GL_KERNEL_DX_DMA, fn, dim3((unsigned)(8LL * k.FR * k.QL * (two ? k.n_tc / 2 : k.n_tc))), dim3(64), 0,
                s, k);
      GL_CHECK_LAUNCH();
      return 0;
    }
  }
  auto fn = dx_kernel<K, T>;
  GL_LAUNCH(GL_KERNEL_DX, fn, dim3((unsigned)(8LL * k.FR * k.QL * k.n_tc)), dim3(64), 0, s, k);
  GL_CHECK_LAUNCH();
  return 0;
}

template <int K>
static int launch_dx_k(int T, const DxK& k, hipStream_t s, bool dma) {
  return T == 1 ? launch_dx_kt<K, 1>(k, s, dma) : (T == 2 ? launch_dx_kt<K, 2>(k, s, dma) : launch_dx_kt<K, 4>(k, s, dma));
}

// dma: the LDS-copy kernel (8 waves per SIMD) for short segments; long segments (narrow pool
// windows) keep dx_kernel, whose 6 waves per SIMD thrash the L2 less when every wave streams
// long runs of many units (C3: 15.5 ms against 20.5, with 45% against 27% L2 hits)
static int launch_dx(int K, int T, const DxK& k, hipStream_t s, bool dma) {
  return K == 8 ? launch_dx_k<8>(T, k, s, dma) : launch_dx_k<16>(T, k, s, dma);
}

template <int K, int ACT, int OP, int PI = -1>
static int launch_bwd_smooth_k(const BsK& k, hipStream_t s) {
  // the power mean with an integer p: p as a literal (C2 recompute 42.1 -> 35.6 ms per 128-token
  // chunk at p = 2)
  if constexpr (OP == SM_POW && PI < 0) {
    switch (k.pint) {
      case 1: return launch_bwd_smooth_k<K, ACT, OP, 1>(k, s);
      case 2: return launch_bwd_smooth_k<K, ACT, OP, 2>(k, s);
      case 4: return launch_bwd_smooth_k<K, ACT, OP, 4>(k, s);
      case 8: return launch_bwd_smooth_k<K, ACT, OP, 8>(k, s);
      default: return launch_bwd_smooth_k<K, ACT, OP, 0>(k, s);
    }
  }
  // neurons per lane: the plan's (its cpg chunks of 64 NPL slots cover every pool exactly)
  constexpr int NPL = smooth_npl(K), WAVES = 8, SB = smooth_sb(K);
  auto fn = k.D <= XTILE_DB ? bwd_smooth_kernel<K, NPL, WAVES, ACT, OP, true, false, SB, PI>
                            : (k.D <= XTILE_SB ? bwd_smooth_kernel<K, NPL, WAVES, ACT, OP, false, false, SB, PI>
                                               : bwd_smooth_kernel<K, NPL, WAVES, ACT, OP, false, true, SB, PI>);
  GL_LAUNCH(GL_KERNEL_BWD_W, fn, dim3((unsigned)ceil_div(k.n_chunks, WAVES)), dim3(WAVES * 64), 0, s, k);
  GL_CHECK_LAUNCH();
  return 0;
}

template <int K, int OP>
static int launch_bwd_smooth_op(int act, const BsK& k, hipStream_t s) {
  if (act == GL_ACT_GELU) return launch_bwd_smooth_k<K, GL_ACT_GELU, OP>(k, s);
  if constexpr (OP == SM_LIN) return GL_ERR_UNSUPPORTED;  // relu / identity sum and mean take the mask path
  else return act == GL_ACT_RELU ? launch_bwd_smooth_k<K, GL_ACT_RELU, OP>(k, s) : launch_bwd_smooth_k<K, GL_ACT_IDENTITY, OP>(k, s);
}

template <int K>
static int launch_bwd_smooth_kk(int pool, int act, const BsK& k, hipStream_t s) {
  if (pool == GL_POOL_POWER) return launch_bwd_smooth_k<K, GL_ACT_RELU, SM_POW>(k, s);
  if (pool == GL_POOL_LME) return launch_bwd_smooth_op<K, SM_LME>(act, k, s);
  if (pool == GL_POOL_SOFTMAX) return launch_bwd_smooth_op<K, SM_SW>(act, k, s);
  return launch_bwd_smooth_op<K, SM_LIN>(act, k, s);
}

template <int K, int T>
static int launch_dx_dense_kt(const DxK& k, const float* dz, hipStream_t s) {
  GL_LAUNCH(GL_KERNEL_DX_DENSE, (dx_dense_kernel<K, T>), dim3((unsigned)(8LL * k.FR * k.QL * k.n_tc)), dim3(64), 0, s, k,
            dz);
  GL_CHECK_LAUNCH();
  return 0;
}

static int launch_dx_dense(int K, int T, const DxK& k, const float* dz, hipStream_t s) {
  if (K == 8) return T == 1 ? launch_dx_dense_kt<8, 1>(k, dz, s) : (T == 2 ? launch_dx_dense_kt<8, 2>(k, dz, s) : launch_dx_dense_kt<8, 4>(k, dz, s));
  return T == 1 ? launch_dx_dense_kt<16, 1>(k, dz, s) : (T == 2 ? launch_dx_dense_kt<16, 2>(k, dz, s) : launch_dx_dense_kt<16, 4>(k, dz, s));
}

static float smooth_scale_b(int pool, float param) {
  const float log2e = 1.4426950408889634f;
  return pool == GL_POOL_LME ? log2e / param : (pool == GL_POOL_SOFTMAX ? log2e * param : 1.f);
}

}  // namespace gl

using namespace gl;

// Average edges per dX segment (one unit's edges into FW features): S K FW / (inputs a unit
// reaches), the pool window's width when the layer has windows (a->win), else D.  Short segments
// (C2: 16, C4: 8, C5: 16) run the LDS-copy dX kernel; a segment of a 256-wide window holds 256.
static bool dx_short_segments(const GlBwdArgs* a) {
  const long long reach = a->win && a->win_width > 0 && a->win_width < a->D ? a->win_width : a->D;
  return (long long)a->S * a->K * FW < 64 * reach;
}

extern "C" int gl_bwd_workspace(const GlBwdArgs* a, size_t* bytes) {
  if (!a || !bytes) return GL_ERR_ARG;
  GL_TRY(check_layer(a->B, a->D, a->G, a->S, a->K, a->act, a->pool, a->X, a->idx, a->W, a->bias, a->counts,
                     a->x_dtype, a->w_dtype));
  const bool smooth = dense_dz(a->pool, a->act);
  BwdPlan q = bwd_plan(a->B, a->D, a->G, a->S, a->K, smooth, a->dz_budget);
  GL_TRY(check_topk(a->pool, a->topk, a->S));
  GL_TRY(check_rec_shift(a->rec_shift, a->S, a->sched));
  GL_TRY(check_smooth(a->pool, a->pool_param, a->act));
  int32_t sps = a->sps, gs = a->gs;
  GL_TRY(check_geometry(a->G, a->S, &sps, &gs));
  if (sps > 1 && a->rec_shift > 0) return GL_ERR_UNSUPPORTED;
  // max / top-k pooling: the transposed selected slots, laid out like c1t (times k for top-k);
  // smooth pools: c2t and c3t beside c1t
  const size_t kpe = a->pool == GL_POOL_TOPK_MEAN ? (size_t)a->topk : (a->pool == GL_POOL_MAX ? 1 : 0);
  *bytes = q.xt_bytes + q.c1_bytes + q.mask_bytes + q.part_bytes + kpe * q.c1_bytes + q.dz_bytes +
           (smooth ? 2 * q.c1_bytes : 0);
  return 0;
}

extern "C" int gl_bwd(const GlBwdArgs* a, void* stream) {
  if (!a || !a->g_pre || !a->dW || !a->db || !a->dX || !a->edges) return GL_ERR_ARG;
  if (a->sched && a->K != 8) return GL_ERR_UNSUPPORTED;
  const bool sel = a->pool == GL_POOL_MAX || a->pool == GL_POOL_TOPK_MEAN;
  if (sel != (a->winner != nullptr)) return GL_ERR_ARG;  // selected slots exactly for max / top-k
  if (a->winner && a->S >= (1 << 21)) return GL_ERR_UNSUPPORTED;  // the event sort keys hold slot << 11
  if (a->relu_mask && !relu_mask_layer(a->act, a->pool, a->K, a->rec_shift, a->x_dtype, a->D)) return GL_ERR_ARG;
  size_t need = 0;
  GL_TRY(gl_bwd_workspace(a, &need));
  if (!a->ws || a->ws_bytes < need) return GL_ERR_WORKSPACE;
  EdgeHeader h;
  size_t edge_bytes = 0;
  edge_layout(a->D, a->G, a->S, a->K, &h, &edge_bytes);
  if (a->edges_bytes < edge_bytes) return GL_ERR_EDGES;
  hipStream_t s = (hipStream_t)stream;
  const bool smooth = dense_dz(a->pool, a->act);
  if (is_smooth(a->pool) && (!a->pre && !(a->pool == GL_POOL_LME && a->lse))) return GL_ERR_ARG;  // coefficients need pre
  if (a->pool == GL_POOL_SOFTMAX && !a->lse) return GL_ERR_ARG;
  BwdPlan q = bwd_plan(a->B, a->D, a->G, a->S, a->K, smooth, a->dz_budget);
  const int sps = a->sps > 1 ? a->sps : 1, gs = a->sps > 1 ? a->gs : a->S;  // checked by gl_bwd_workspace
  char* ws = (char*)a->ws;
  float4* xt = (float4*)ws;
  float* c1t = (float*)(ws + q.xt_bytes);
  uint32_t* mask = (uint32_t*)(ws + q.xt_bytes + q.c1_bytes);
  float* part = (float*)(ws + q.xt_bytes + q.c1_bytes + q.mask_bytes);
  int32_t* wint = a->winner ? (int32_t*)(ws + q.xt_bytes + q.c1_bytes + q.mask_bytes + q.part_bytes) : nullptr;
  const char* eb = (const char*)a->edges;
  // W and bias in their stored dtype (bf16: widened in the kernels)
  const float* W = (const float*)a->W;
  const float* bias = (const float*)a->bias;
  const int wbf = a->w_dtype == GL_DTYPE_BF16;

  for (int b0 = 0; b0 < a->B; b0 += q.bc_max) {
    const int Bc = a->B - b0 < q.bc_max ? a->B - b0 : q.bc_max;
    const int n_tiles = ceil_div(Bc, BT);
    const int T = dx_slots(Bc);
    const int cap = dx_cap(Bc);
    // the dense dW pass over full tiles of 4097..8192 inputs reads two-token tiles (two 64-KiB buffers)
    int ww = 0, npw = 0;
    const bool dense = !smooth && !a->winner;
    // the staged windows cover the pools of one workgroup: size them for the dW launch that runs
    // (16 waves with the forward's ReLU bits, else bwd_waves)
    const int dw_waves = a->relu_mask && a->K == 8 ? BWD_FM_WIN_WAVES : q.waves;
    // bf16 X staged in pool windows keeps its bf16 values (8-byte inputs, windows from an even input),
    // as the forward's windows do: with the forward's ReLU bits (159 VGPRs) or identity neurons;
    // the ReLU recompute at 12 waves would spill 60 bytes per lane, and keeps fp32 windows
    const bool xbw = dense && a->x_dtype == GL_DTYPE_BF16 && a->D % 2 == 0 && a->D <= 2 * XTILE_DB &&
                     (a->relu_mask || a->act == GL_ACT_IDENTITY);
    const bool win = dense && window_staging(a->win, a->win_width, a->D, dw_waves, q.cpg, a->G, &ww, &npw, WS_SLOTS,
                                             xbw ? 8 : 16);
    const bool wide = dense && !win && tiles_of_two(a->D);
    // bf16 X keeps its bf16 values, 4 tokens per 8-byte slot (C4 dW 114.3 -> 90.2 ms against
    // two-token fp32 tiles: half the gathers and tile overheads per token for one widening per value)
    const bool xb = (wide && a->x_dtype == GL_DTYPE_BF16) || (win && xbw);
    const int tb = wide && !xb ? 2 : BT;
    if (xb)
      GL_TRY(launch_tile_x_bf16x4(a->X, a->sxb, a->B, a->D, b0, n_tiles, xt, s));
    else
      GL_TRY(launch_tile_x(a->X, a->sxb, a->x_dtype, a->B, a->D, b0, n_tiles * BT / tb, xt, s, tb));
    if (smooth) {  // coefficients, recompute pass (dW, db, dz), dX from dz (smooth pools, GELU sum / mean)
      float* c2t = (float*)(ws + q.xt_bytes + q.c1_bytes + q.part_bytes);
      float* c3t = (float*)((char*)c2t + q.c1_bytes);
      float* dz = (float*)((char*)c3t + q.c1_bytes);
      const float scale = smooth_scale_b(a->pool, a->pool_param);
      GL_LAUNCH(GL_KERNEL_C1T, coef_smooth_kernel, dim3((unsigned)ceil_div(a->G, 32), (unsigned)ceil_div(cap, 32)),
                dim3(256), 0, s, a->g_pre, a->pre, a->lse, a->counts, c1t, c2t, c3t, a->G, b0, Bc, cap, a->pool, scale);
      GL_CHECK_LAUNCH();
      const int pint = a->pool == GL_POOL_POWER &&
                               (a->pool_param == 1.f || a->pool_param == 2.f || a->pool_param == 4.f || a->pool_param == 8.f)
                           ? (int)a->pool_param
                           : 0;
      BsK bk{xt, a->idx, W, bias, a->counts, c1t, c2t, c3t, a->dW, a->db, dz, a->sched, q.n_chunks, a->D,
             a->S, q.cpg, n_tiles, cap, ceil_div(a->S, SCHED_WIN), a->rec_shift, scale, a->pool_param, pint,
             sps, gs};
      bk.wbf = wbf;
      GL_TRY(a->K == 8 ? launch_bwd_smooth_kk<8>(a->pool, a->act, bk, s) : launch_bwd_smooth_kk<16>(a->pool, a->act, bk, s));
      const long long NS = (long long)a->G * a->S;
      const int Td = T;
      DxK dk{(const uint32_t*)(eb + h.off_rec), (const uint32_t*)(eb + h.off_seg_ptr),
             (const int32_t*)(eb + h.off_seg_unit), (const uint32_t*)(eb + h.off_seg_begin), c1t, nullptr, W, part,
             NS, a->D, a->S, q.P, q.U, q.QL, q.UQs, q.FR, cap, cap / (64 * Td), sps, gs};
      dk.wbf = wbf;
      for (int ql0 = 0; ql0 < q.QLs; ql0 += q.QL) {  // passes of QL unit ranges per XCD
        dk.ql0 = ql0;
        GL_TRY(launch_dx_dense(a->K, Td, dk, dz, s));
        GL_LAUNCH(GL_KERNEL_DX_REDUCE, dx_reduce_kernel, dim3((unsigned)ceil_div(a->D, 32), (unsigned)ceil_div(Bc, 32)),
                  dim3(256), 0, s, part, a->dX, a->D, cap, q.Q, b0, Bc, ql0 > 0 ? 1 : 0);
        GL_CHECK_LAUNCH();
      }
      continue;
    }
    const int kpe = a->pool == GL_POOL_TOPK_MEAN ? a->topk : 1;
    GL_LAUNCH(GL_KERNEL_C1T, c1t_kernel, dim3((unsigned)ceil_div(a->G, 32), (unsigned)ceil_div(cap, 32)), dim3(256), 0, s,
                       a->g_pre, a->counts, c1t, a->G, b0, Bc, cap, a->pool, a->topk, kpe == 1 ? a->winner : nullptr,
                       wint);
    GL_CHECK_LAUNCH();
    if (a->winner) {  // max / top-k pooling: selection events (gl_max_bwd.hip), no dense pass
      if (kpe > 1) {
        GL_LAUNCH(GL_KERNEL_C1T, events_transpose_kernel, dim3((unsigned)ceil_div((long long)a->G * cap * kpe, 256)),
                  dim3(256), 0, s, a->winner, wint, a->G, b0, Bc, cap, kpe);
        GL_CHECK_LAUNCH();
      }
      MaxEvKArgs ev{xt, a->idx, W, bias, a->counts, c1t, wint, a->g_pre, a->winner, a->dW, a->db, a->dX,
                    a->D, a->G, a->S, cap, Bc, b0, kpe, a->rec_shift, a->pool == GL_POOL_TOPK_MEAN, sps, gs};
      ev.wbf = wbf;
      GL_TRY(launch_max_events(a->K, a->act, ev, s));
      continue;
    }
    const long long NS = (long long)a->G * a->S;
    BwK bk{xt, a->idx, W, bias, a->counts, c1t, a->dW, a->db, mask, a->sched, nullptr, q.n_chunks, NS,
           a->D, a->S, q.cpg, n_tiles * BT / tb, cap, 2 * T, ceil_div(a->S, SCHED_WIN), a->G, ww, npw, a->rec_shift,
           sps, gs, tb, xb ? 1 : 0};
    bk.wbf = wbf;
    if (win) bk.win = a->win;
    if (a->relu_mask) {  // the forward's bits, per 4-token tile of the batch
      if (tb != BT) return GL_ERR_ARG;
      bk.fm = (const uint16_t*)a->relu_mask;
      bk.fm_tiles = ceil_div(a->B, BT);
      bk.fm_t0 = b0 / BT;
    }
    GL_TRY(launch_bwd_w_any(a->K, a->act, bk, s));
    DxK dk{(const uint32_t*)(eb + h.off_rec), (const uint32_t*)(eb + h.off_seg_ptr),
           (const int32_t*)(eb + h.off_seg_unit), (const uint32_t*)(eb + h.off_seg_begin), c1t, mask, W, part,
           NS, a->D, a->S, q.P, q.U, q.QL, q.UQ, q.FR, cap, cap / (64 * T), sps, gs};
    dk.wbf = wbf;
    GL_TRY(launch_dx(a->K, T, dk, s, dx_short_segments(a)));
    GL_LAUNCH(GL_KERNEL_DX_REDUCE, dx_reduce_kernel, dim3((unsigned)ceil_div(a->D, 32), (unsigned)ceil_div(Bc, 32)), dim3(256), 0,
                       s, part, a->dX, a->D, cap, q.Q, b0, Bc, 0);
    GL_CHECK_LAUNCH();
  }
  return 0;
}
