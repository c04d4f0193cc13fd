// Forward: fused sparse projection -> activation -> pool (sum / mean, max, top-k mean), neuron-stationary.
//
// Each wave owns a "chunk": up to 64*NPL consecutive slots of one group, NPL neurons per lane
// (slot s_lo + j*64 + lane, or the gather schedule's permutation of the chunk's 128-slot
// windows).  Index records, weights and bias of the chunk are loaded into VGPRs
// once; the wave then streams every token tile of X through LDS (4 tokens per 16-byte slot,
// feature-major), gathers one slot per (neuron, k) with ds_read_b128, accumulates z in fp32,
// applies the activation and reduces the chunk's per-token sum across the wave.  The hidden
// tensor [B, H] never exists; only per-(chunk, token) partial sums are written and a finalize
// kernel merges the chunks of a group in a fixed order (reference: fwd_pool_kernel +
// merge_finalize, sparse_pooling/kernels/triton_fused.py:289-358, kernels/ops.py:182-199).
#include <mutex>
#include <type_traits>

#include "gl_common.h"
#include "gl_internal.h"

namespace gl {

// X [B, D] (fp32 | bf16, row stride sxb) -> XT [n_tiles][D][TB] fp32 (TB = 4 tokens per 16-byte
// slot, or 2 per 8-byte slot); tokens >= B are zero.
template <typename XT, int TB>
__global__ void __launch_bounds__(256) tile_x_kernel(const XT* __restrict__ X, long long sxb, int B, int D, int b0,
                                                     int n_tiles, float* __restrict__ out) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  long long total = (long long)n_tiles * D;
  if (i >= total) return;
  int t = (int)(i / D), d = (int)(i % D);
  float v[TB];
#pragma unroll
  for (int j = 0; j < TB; ++j) {
    int b = b0 + t * TB + j;
    v[j] = b < B ? load_x(X, (long long)b * sxb + d) : 0.f;
  }
  if constexpr (TB == 4) reinterpret_cast<float4*>(out)[i] = make_float4(v[0], v[1], v[2], v[3]);
  else reinterpret_cast<float2*>(out)[i] = make_float2(v[0], v[1]);
}

// bf16 X [B, D] -> XT [n_tiles][D] of 4 tokens as raw bf16 bits in 8 bytes: word 0 = token 1 << 16 |
// token 0, word 1 = token 3 << 16 | token 2 (tokens >= B are +0).  The kernels widen each value
// with one shift or mask, which is exact.
__global__ void __launch_bounds__(256) tile_x_bf16x4_kernel(const unsigned short* __restrict__ X, long long sxb, int B,
                                                            int D, int b0, int n_tiles, uint2* __restrict__ out) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  long long total = (long long)n_tiles * D;
  if (i >= total) return;
  int t = (int)(i / D), d = (int)(i % D);
  unsigned v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int b = b0 + t * 4 + j;
    v[j] = b < B ? (unsigned)X[(long long)b * sxb + d] : 0u;
  }
  out[i] = make_uint2(v[1] << 16 | v[0], v[3] << 16 | v[2]);
}

template <int TB>
static int launch_tile_x_tb(const void* X, long long sxb, int x_dtype, int B, int D, int b0, int n_tiles, float* xt,
                            hipStream_t s) {
  long long total = (long long)n_tiles * D;
  dim3 grid((unsigned)ceil_div(total, 256));
  if (x_dtype == GL_DTYPE_F32)
    GL_LAUNCH(GL_KERNEL_TILE_X, (tile_x_kernel<float, TB>), grid, dim3(256), 0, s, (const float*)X, sxb, B, D, b0,
              n_tiles, xt);
  else
    GL_LAUNCH(GL_KERNEL_TILE_X, (tile_x_kernel<__hip_bfloat16, TB>), grid, dim3(256), 0, s, (const __hip_bfloat16*)X,
              sxb, B, D, b0, n_tiles, xt);
  GL_CHECK_LAUNCH();
  return 0;
}

// bf16 X only: 4-token tiles of raw bf16 (8-byte slots)
int launch_tile_x_bf16x4(const void* X, long long sxb, int B, int D, int b0, int n_tiles, void* xt,
                                hipStream_t s) {
  long long total = (long long)n_tiles * D;
  dim3 grid((unsigned)ceil_div(total, 256));
  GL_LAUNCH(GL_KERNEL_TILE_X, tile_x_bf16x4_kernel, grid, dim3(256), 0, s, (const unsigned short*)X, sxb, B, D, b0,
            n_tiles, (uint2*)xt);
  GL_CHECK_LAUNCH();
  return 0;
}

int launch_tile_x(const void* X, long long sxb, int x_dtype, int B, int D, int b0, int n_tiles, float4* xt,
                  hipStream_t s, int tb) {
  return tb == 2 ? launch_tile_x_tb<2>(X, sxb, x_dtype, B, D, b0, n_tiles, (float*)xt, s)
                 : launch_tile_x_tb<4>(X, sxb, x_dtype, B, D, b0, n_tiles, (float*)xt, s);
}

struct FwdK {
  const float4* xt;       // [n_tiles][D] float4
  const int32_t* idx;
  const float* W;
  const float* bias;
  const int32_t* counts;
  float* part;            // [n_chunks][b_pad]
  int* pslot;             // max / top-k pooling: [n_chunks][b_pad][kp] slot of each partial candidate
  int topk;               // top-k pooling: k (candidates per chunk and token)
  const uint32_t* sched;  // gather schedule or null
  const uint32_t* win;    // per-pool window starts (window staging) or null
  long long n_chunks;
  int D, S, cpg, n_tiles, b_pad, nwin;
  int G, ww, npw;         // window staging: pools, padded window width, pools per workgroup
  int rs;                 // log2 slots per shared index record
  float scale, pparam;    // smooth pools: u = a * scale (LogMeanExp / softmax-weighted); p (power mean)
  int pint;               // power mean: p when it is 1, 2, 4 or 8 (exact products), else 0
  int sps, gs;            // pool geometry (pool_base): shards per group and group stride in slots
  int tb;                 // tokens per tile: 4, or 2 (two-token tiles; n_tiles counts those)
  int ws_small;           // window staging in workgroups of half the waves (two per CU, 64 KiB of stages)
  int xb;                 // 4-token tiles of raw bf16 (8-byte slots; bf16 X, sum / mean)
  int wbf;                // W and bias stored as bf16 (widened in the kernel)
  uint16_t* fm;           // ReLU bits for the backward ([n_chunks][fm_tiles][64] 16-bit words) or null
  int fm_tiles, fm_t0;    // 4-token tiles of the whole batch; the pass's first tile
};

// ReLU activation bits of a lane's neurons for the backward, shifted in as they are decided: after
// a tile, bit 15 - (4 j + i) of the 16-bit word is token i of the tile for the lane's neuron j.  The
// kernel stores each tile's word (64 lanes x 2 bytes, one coalesced store), so no state is held
// across tiles.  With them the backward's dW pass skips the recompute of z.  NoBits is the sink of
// the kernels that keep none.
struct NoBits {};
struct ReluBits {
  unsigned bits;
};
template <typename MB>
__device__ __forceinline__ void relu_bits(MB&, int, float, float, float, float) {}
// bits = 2 bits + (a > 0): the compare's lane mask is the carry-in of one add (two VALU per bit
// where compare, select and or took three), issued here rather than sunk to the end of the tile,
// which kept 16 activations live and spilled at 128 VGPRs
__device__ __forceinline__ void relu_bit(unsigned& bits, float a) {
  unsigned long long c;
  asm volatile("v_cmp_lt_f32_e64 %1, 0, %2\n\tv_addc_co_u32_e64 %0, %1, %0, %0, %1"
               : "+v"(bits), "=&s"(c)
               : "v"(a));
}
__device__ __forceinline__ void relu_bits(ReluBits& m, int, float a0, float a1, float a2, float a3) {
  relu_bit(m.bits, a0);
  relu_bit(m.bits, a1);
  relu_bit(m.bits, a2);
  relu_bit(m.bits, a3);
}

// One token tile (4 tokens per 16-byte LDS entry at xsb): z = bias + sum_k w * x[idx], activation,
// pooled over the wave's neurons and lanes (wave_sum4; lanes 0-3 store the 4 token sums).  The
// first RA LDS reads of neuron j + 1 are issued before the arithmetic of neuron j, so up to K + RA
// reads are in flight per wave (the compiler's own schedule keeps two).
template <int K, int NPL, int ACT, bool FAR, int RA = (K == 8 ? 4 : 8), typename SRC = const char*,
          typename MB = NoBits>
__device__ __forceinline__ void fwd_tile(SRC xsb, const unsigned (&addr)[NPL][K], const float (&w)[NPL][K],
                                         const float (&bias)[NPL], float* out, bool store, int lane, MB& mb) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
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
    float z0 = bias[j], z1 = bias[j], z2 = bias[j], z3 = bias[j];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      z0 = __builtin_fmaf(xc[k].x, w[j][k], z0);
      z1 = __builtin_fmaf(xc[k].y, w[j][k], z1);
      z2 = __builtin_fmaf(xc[k].z, w[j][k], z2);
      z3 = __builtin_fmaf(xc[k].w, w[j][k], z3);
    }
    z0 = act_f<ACT>(z0);
    z1 = act_f<ACT>(z1);
    z2 = act_f<ACT>(z2);
    z3 = act_f<ACT>(z3);
    relu_bits(mb, j, z0, z1, z2, z3);
    a0 += z0;
    a1 += z1;
    a2 += z2;
    a3 += z3;
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xc[k] = xn[k];
    }
  }
  const float tot = wave_sum4(a0, a1, a2, a3, lane);
  if (store && lane < 4) out[wave_sum4_token(lane)] = tot;  // 4 lanes, 16 contiguous bytes
}

// The sum / mean tile over a 4-token tile of raw bf16 values (8-byte slots, ds_read_b64): the gathers
// keep the packed words (the read-ahead holds 2 registers per slot, not 4) and each value is
// widened (shift or mask: exact) right before its FMA.  The arithmetic is fwd_tile's.
template <int K, int NPL, int ACT, bool FAR, int RA = (K == 8 ? 4 : 8), typename MB = NoBits>
__device__ __forceinline__ void fwd_tile_bf4(const char* xsb, const unsigned (&addr)[NPL][K], const float (&w)[NPL][K],
                                             const float (&bias)[NPL], float* out, bool store, int lane, MB& mb) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  uint2 xc[K];
  auto ld = [&](unsigned a) {
    if constexpr (FAR) asm volatile("" : "+v"(a));
    return *reinterpret_cast<const uint2*>(xsb + a);
  };
#pragma unroll
  for (int k = 0; k < RA; ++k) xc[k] = ld(addr[0][k]);
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
#pragma unroll
    for (int k = RA; k < K; ++k) xc[k] = ld(addr[j][k]);
    uint2 xn[RA];
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xn[k] = ld(addr[j + 1][k]);
    }
    __builtin_amdgcn_sched_barrier(0);
    float z0 = bias[j], z1 = bias[j], z2 = bias[j], z3 = bias[j];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      z0 = __builtin_fmaf(__uint_as_float(xc[k].x << 16), w[j][k], z0);
      z1 = __builtin_fmaf(__uint_as_float(xc[k].x & 0xffff0000u), w[j][k], z1);
      z2 = __builtin_fmaf(__uint_as_float(xc[k].y << 16), w[j][k], z2);
      z3 = __builtin_fmaf(__uint_as_float(xc[k].y & 0xffff0000u), w[j][k], z3);
    }
    z0 = act_f<ACT>(z0);
    z1 = act_f<ACT>(z1);
    z2 = act_f<ACT>(z2);
    z3 = act_f<ACT>(z3);
    relu_bits(mb, j, z0, z1, z2, z3);
    a0 += z0;
    a1 += z1;
    a2 += z2;
    a3 += z3;
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xc[k] = xn[k];
    }
  }
  const float tot = wave_sum4(a0, a1, a2, a3, lane);
  if (store && lane < 4) out[wave_sum4_token(lane)] = tot;
}

// The sum / mean tile over a two-token tile (8-byte slots, ds_read_b64); lanes 0-1 store.
template <int K, int NPL, int ACT, bool FAR, int RA = (K == 8 ? 4 : 8)>
__device__ __forceinline__ void fwd_tile2(const char* xsb, const unsigned (&addr)[NPL][K], const float (&w)[NPL][K],
                                          const float (&bias)[NPL], float* out, bool store, int lane) {
  float a0 = 0.f, a1 = 0.f;
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
    z0 = act_f<ACT>(z0);
    z1 = act_f<ACT>(z1);
    a0 += z0;
    a1 += z1;
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xc[k] = xn[k];
    }
  }
  const float tot = wave_sum2(a0, a1, lane);
  if (store && lane < 2) out[lane] = tot;  // 2 lanes, 8 contiguous bytes
}

// Max pooling tile: per token the largest act(z) of the wave's neurons and its pool slot (the
// smaller slot on ties), reduced over the lanes by wave_max4; lanes 0-3 store value and slot.
// Padded slots carry z = -inf (bias -inf, weights 0) and slots >= n_g, so they never win: with
// relu they tie at 0 with a valid slot and lose on the slot.
template <int K, int NPL, int ACT, bool FAR, int RA = (K == 8 ? 4 : 8), typename SRC = const char*>
__device__ __forceinline__ void fwd_tile_max(SRC xsb, const unsigned (&addr)[NPL][K], const float (&w)[NPL][K],
                                             const float (&bias)[NPL], const int (&slot)[NPL], float* out, int* oslot,
                                             bool store, int lane) {
  float m0 = -__builtin_inff(), m1 = m0, m2 = m0, m3 = m0;
  int s0 = 0x7fffffff, s1 = s0, s2 = s0, s3 = s0;
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
    float z0 = bias[j], z1 = bias[j], z2 = bias[j], z3 = bias[j];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      z0 = __builtin_fmaf(xc[k].x, w[j][k], z0);
      z1 = __builtin_fmaf(xc[k].y, w[j][k], z1);
      z2 = __builtin_fmaf(xc[k].z, w[j][k], z2);
      z3 = __builtin_fmaf(xc[k].w, w[j][k], z3);
    }
    z0 = act_f<ACT>(z0);
    z1 = act_f<ACT>(z1);
    z2 = act_f<ACT>(z2);
    z3 = act_f<ACT>(z3);
    // A lane's neurons 2i and 2i + 1 share a 128-slot window (sched_slot), later pairs lie in later
    // windows: slot[2i] exceeds every slot before it, so a strict compare keeps ties on the
    // smaller slot there; inside a pair the order is free and the full pair compare decides.
    if (j == 0) {
      m0 = z0, m1 = z1, m2 = z2, m3 = z3;
      s0 = s1 = s2 = s3 = slot[0];
    } else if (j % 2 == 0) {
      const bool t0 = z0 > m0, t1 = z1 > m1, t2 = z2 > m2, t3 = z3 > m3;
      m0 = t0 ? z0 : m0, s0 = t0 ? slot[j] : s0;
      m1 = t1 ? z1 : m1, s1 = t1 ? slot[j] : s1;
      m2 = t2 ? z2 : m2, s2 = t2 ? slot[j] : s2;
      m3 = t3 ? z3 : m3, s3 = t3 ? slot[j] : s3;
    } else {
      vmax_pair(m0, s0, z0, slot[j]);
      vmax_pair(m1, s1, z1, slot[j]);
      vmax_pair(m2, s2, z2, slot[j]);
      vmax_pair(m3, s3, z3, slot[j]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xc[k] = xn[k];
    }
  }
  float m;
  int sl;
  wave_max4(m0, m1, m2, m3, s0, s1, s2, s3, lane, m, sl);
  if (store && lane < 4) {
    out[wave_sum4_token(lane)] = m;
    oslot[wave_sum4_token(lane)] = sl;
  }
}

// Top-k candidates as 64-bit keys, one unsigned compare per ordering decision.  The high word
// maps the fp32 value to an unsigned integer of the same order (negative values bit-inverted,
// the others with the sign bit set; -0 is first made +0, so equal values compare equal); the low
// word is ~slot, so that of two equal values the smaller slot ranks higher.  Slots are distinct
// within a wave, so keys never tie.  The finalize merges the chunk lists with the same keys, so the
// selection does not depend on how a pool is split into chunks.
using cand_t = unsigned long long;
__device__ __forceinline__ cand_t cand_key(float v, unsigned nslot) {
  // NaN of either sign ranks above every number (torch.sort's order); -0 is made +0
  const unsigned b = __builtin_isnan(v) ? 0x7fc00000u : __float_as_uint(v + 0.f);
  const unsigned o = b ^ ((unsigned)((int)b >> 31) | 0x80000000u);
  return ((cand_t)o << 32) | nslot;
}
__device__ __forceinline__ float cand_value(cand_t c) {
  const unsigned o = (unsigned)(c >> 32);
  return __uint_as_float((o & 0x80000000u) ? (o ^ 0x80000000u) : ~o);
}
// the key of (-inf, slot 0x7fffffff): below every candidate a wave holds
constexpr cand_t CAND_NONE = (0x007fffffull << 32) | 0x80000000u;

// a before b in the best-first order
__device__ __forceinline__ void cand_cmpex(cand_t& a, cand_t& b) {
  const bool swap = b > a;
  const cand_t t = a;
  a = swap ? b : a;
  b = swap ? t : b;
}

// 32-bit wave_max4 (the same reduce-scatter as wave_sum4): every lane ends with the maximum of
// token wave_sum4_token(lane) over the wave
template <int CTRL>
__device__ __forceinline__ unsigned dppu(unsigned v) {
  return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ unsigned umax(unsigned a, unsigned b) { return a > b ? a : b; }
__device__ __forceinline__ unsigned umin(unsigned a, unsigned b) { return a < b ? a : b; }
__device__ __forceinline__ unsigned wave_max4_u32(unsigned a0, unsigned a1, unsigned a2, unsigned a3, int lane) {
  const bool odd = lane & 1, hi = lane & 2;
  const unsigned b0 = umax(odd ? a2 : a0, dppu<0xB1>(odd ? a0 : a2));  // quad_perm(1,0,3,2)
  const unsigned b1 = umax(odd ? a3 : a1, dppu<0xB1>(odd ? a1 : a3));
  unsigned c = umax(hi ? b1 : b0, dppu<0x4E>(hi ? b0 : b1));           // quad_perm(2,3,0,1)
  c = umax(c, dppu<0x124>(c));                                          // row_ror:4
  c = umax(c, dppu<0x128>(c));                                          // row_ror:8
  const auto p16 = __builtin_amdgcn_permlane16_swap(c, c, false, false);
  c = umax(p16[0], p16[1]);
  const auto p32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return umax(p32[0], p32[1]);
}

// Top-k tile (top-k mean pooling, pytorch_reference.py:68-77): per token the k largest raw z of the
// wave's neurons with their slots (ties to the smaller slot), best first.  Every lane sorts its 4
// candidates per token (64-bit keys: value order, then ~slot); then k rounds take the wave's best
// head and drop it from the lane that holds it.  A round finds the best head in two 32-bit steps:
// the largest value order, then among the heads of that value the largest ~slot (the smallest
// slot); the winner is the 64-bit maximum, as one 64-bit reduction would give, at a third of its
// VALU (a 64-bit compare and two selects per reduction step become one v_max_u32).  Lanes 0-3
// store each round's pair; the finalize merges the pool's chunks.
//
// Ranked path (TKW > 0 waves per workgroup, k <= 8): no rounds.  A lower bound of every token's
// k-th largest value: the 8th largest of its 16 lane-quad maxima (16 disjoint sets of candidates,
// so 8 distinct candidates lie at or above it; a bitonic sort across the quads finds it).  The
// candidates at or above the bound (~10 of 256 on random data) are compacted into a
// per-wave LDS list per token (ballot, mbcnt, zero keys to a multiple of 16); each then counts the
// list's larger keys (16-key blocks, all reads of a block in flight together) for its rank and
// stores itself at that position.  Same keys, same order: the output is the rounds' output, bit for
// bit.  A token with more than 64 candidates at the bound (ties, or a chunk of mostly padded slots
// at -inf) sends the tile to the rounds.  At C2 (top-8) the ranked tile took the forward from 68.9
// to 65.5 ms at 8 waves per workgroup, and its 158 VGPRs allow 12 (54.0 ms); the quad-maxima
// bound then took it to 45.4 ms against the smallest maximum of 32-candidate windows (~24
// survivors per token), and ranking the 4 tokens together to 39.1 ms.
// keys per token list: 64, and 2 more so that the 4 tokens' lists start 4 banks apart (the
// 4-token rank reads one 16-byte slot of each list in one ds_read_b128)
constexpr int TK_CAP = 66;
// the lists of a workgroup of TKW waves (one array per kernel, whichever tiles use it)
template <int TKW>
__device__ __forceinline__ cand_t* tk_lists() {
  __shared__ __align__(16) cand_t tkl[TKW * 4 * TK_CAP];
  return tkl;
}
template <int K, int NPL, int ACT, bool FAR, int TKW = 0, int RA = (K == 8 ? 4 : 8), typename SRC = const char*>
__device__ __forceinline__ void fwd_tile_topk(SRC xsb, const unsigned (&addr)[NPL][K], const float (&w)[NPL][K],
                                              const float (&bias)[NPL], const int (&slot)[NPL], float* out, int* oslot,
                                              int k, bool store, int lane) {
  static_assert(NPL == 4, "per-lane candidate lists of 4");
  cand_t c[4][4];  // [token][position]
  float4 xc[K];
#pragma unroll
  for (int k0 = 0; k0 < RA; ++k0) xc[k0] = gather_x<FAR>(xsb, addr[0][k0]);
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
#pragma unroll
    for (int kk = RA; kk < K; ++kk) xc[kk] = gather_x<FAR>(xsb, addr[j][kk]);
    float4 xn[RA];
    if (j + 1 < NPL) {
#pragma unroll
      for (int kk = 0; kk < RA; ++kk) xn[kk] = gather_x<FAR>(xsb, addr[j + 1][kk]);
    }
    __builtin_amdgcn_sched_barrier(0);
    float z0 = bias[j], z1 = bias[j], z2 = bias[j], z3 = bias[j];
#pragma unroll
    for (int kk = 0; kk < K; ++kk) {
      z0 = __builtin_fmaf(xc[kk].x, w[j][kk], z0);
      z1 = __builtin_fmaf(xc[kk].y, w[j][kk], z1);
      z2 = __builtin_fmaf(xc[kk].z, w[j][kk], z2);
      z3 = __builtin_fmaf(xc[kk].w, w[j][kk], z3);
    }
    const unsigned ns = ~(unsigned)slot[j];  // raw z ranks (the activation is the finalize's)
    c[0][j] = cand_key(z0, ns), c[1][j] = cand_key(z1, ns), c[2][j] = cand_key(z2, ns), c[3][j] = cand_key(z3, ns);
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < NPL) {
#pragma unroll
      for (int kk = 0; kk < RA; ++kk) xc[kk] = xn[kk];
    }
  }
  if constexpr (TKW > 0) {
    if (k <= 8) {
      // value-order words of the lane's (unsorted) candidates; the lane's best per token,
      // reduce-scattered to quads as in wave_max4_u32: lane l ends with its quad's maximum for token
      // wave_sum4_token(l)
      unsigned hw[4][4], h[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) hw[t][i] = (unsigned)(c[t][i] >> 32);
        h[t] = umax(umax(hw[t][0], hw[t][1]), umax(hw[t][2], hw[t][3]));
      }
      const bool odd = lane & 1, hi2 = lane & 2;
      const unsigned b0 = umax(odd ? h[2] : h[0], dppu<0xB1>(odd ? h[0] : h[2]));
      const unsigned b1 = umax(odd ? h[3] : h[1], dppu<0xB1>(odd ? h[1] : h[3]));
      unsigned q = umax(hi2 ? b1 : b0, dppu<0x4E>(hi2 ? b0 : b1));
      // bitonic sort (ascending) of each token's 16 quad maxima across the quads (element i = lane
      // bits 2-5; partner i ^ jj = lane ^ 4 jj): the 8th largest ends in quad 8.  Each exchange
      // yields the pair {own, partner} in some order, so min / max of the pair need no direction.
      const int qi = lane >> 2;
#pragma unroll
      for (int kk = 2; kk <= 16; kk <<= 1) {
#pragma unroll
        for (int jj = kk >> 1; jj >= 1; jj >>= 1) {
          unsigned a = q, b;
          if (jj == 8) {
            const auto pr = __builtin_amdgcn_permlane32_swap(q, q, false, false);
            a = pr[0], b = pr[1];
          } else if (jj == 4) {
            const auto pr = __builtin_amdgcn_permlane16_swap(q, q, false, false);
            a = pr[0], b = pr[1];
          } else if (jj == 2) {
            b = dppu<0x128>(q);  // row_ror:8 within a 16-lane row: lane ^ 8
          } else {
            b = (unsigned)__builtin_amdgcn_ds_swizzle((int)q, 0x101f);  // lane ^ 4
          }
          const bool keep_min = ((qi & jj) == 0) == ((qi & kk) == 0);
          q = keep_min ? umin(a, b) : umax(a, b);
        }
      }
      unsigned long long m[4][4];
      int n[4];
      bool over = false;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const unsigned bnd = (unsigned)__builtin_amdgcn_readlane((int)q, 32 + ((t == 1) ? 2 : (t == 2) ? 1 : t));
        n[t] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // any of a lane's 4 candidates may reach the bound
          m[t][i] = __builtin_amdgcn_ballot_w64(hw[t][i] >= bnd);
          n[t] += (int)__builtin_popcountll(m[t][i]);
        }
        over |= n[t] > 64;
      }
      if (!over) {
        cand_t* L = tk_lists<TKW>() + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) * (4 * TK_CAP);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          int base = t * TK_CAP;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (m[t][i] == 0) continue;
            const unsigned pos = __builtin_amdgcn_mbcnt_hi((unsigned)(m[t][i] >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((unsigned)m[t][i], 0u));
            if ((m[t][i] >> lane) & 1) L[base + (int)pos] = c[t][i];
            base += (int)__builtin_popcountll(m[t][i]);
          }
          // zero keys (below every key) up to the next 32-key block
          const int nb = (n[t] + 15) & ~15;
          if (lane >= n[t] && lane < nb) L[t * TK_CAP + lane] = 0ull;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (n[0] <= 16 && n[1] <= 16 && n[2] <= 16 && n[3] <= 16) {
          // every list fits one 16-key block: lanes 16 t .. 16 t + 15 rank token t's list together
          const int tl = lane >> 4, il = lane & 15;
          const int nt = tl == 0 ? n[0] : (tl == 1 ? n[1] : (tl == 2 ? n[2] : n[3]));
          const cand_t* Lt = L + tl * TK_CAP;
          const cand_t mine = Lt[il];
          ulonglong2 kv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) kv[i] = *reinterpret_cast<const ulonglong2*>(Lt + 2 * i);
          unsigned r = 0;
#pragma unroll
          for (int i = 0; i < 8; ++i) r += (kv[i].x > mine) + (kv[i].y > mine);
          if (store && il < nt && r < (unsigned)k) {
            out[tl * k + (int)r] = cand_value(mine);
            oslot[tl * k + (int)r] = (int)~(unsigned)mine;
          }
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const cand_t* Lt = L + t * TK_CAP;
            const cand_t mine = Lt[lane < n[t] ? lane : 0];
            unsigned r = 0;
            for (int j0 = 0; j0 < n[t]; j0 += 16) {  // blocks of 16 keys, all reads issued first
              ulonglong2 kv[8];
#pragma unroll
              for (int i = 0; i < 8; ++i) kv[i] = *reinterpret_cast<const ulonglong2*>(Lt + j0 + 2 * i);
#pragma unroll
              for (int i = 0; i < 8; ++i) r += (kv[i].x > mine) + (kv[i].y > mine);
            }
            if (store && lane < n[t] && r < (unsigned)k) {
              out[t * k + (int)r] = cand_value(mine);
              oslot[t * k + (int)r] = (int)~(unsigned)mine;
            }
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the next tile's lists overwrite these
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        return;
      }
    }
  }
  unsigned o[4][4], sl[4][4];  // the sorted lists as value-order and ~slot words
#pragma unroll
  for (int t = 0; t < 4; ++t) {  // sorting network for 4
    cand_cmpex(c[t][0], c[t][1]);
    cand_cmpex(c[t][2], c[t][3]);
    cand_cmpex(c[t][0], c[t][2]);
    cand_cmpex(c[t][1], c[t][3]);
    cand_cmpex(c[t][1], c[t][2]);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[t][i] = (unsigned)(c[t][i] >> 32), sl[t][i] = (unsigned)c[t][i];
  }
  constexpr unsigned NONE_O = (unsigned)(CAND_NONE >> 32), NONE_S = (unsigned)CAND_NONE;
  const int tok = wave_sum4_token(lane);
  for (int r = 0; r < k; ++r) {
    const unsigned mo = wave_max4_u32(o[0][0], o[1][0], o[2][0], o[3][0], lane);
    unsigned mot[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)  // lanes 0, 2, 1, 3 hold tokens 0, 1, 2, 3
      mot[t] = (unsigned)__builtin_amdgcn_readlane((int)mo, (t == 1) ? 2 : (t == 2) ? 1 : t);
    unsigned es[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) es[t] = o[t][0] == mot[t] ? sl[t][0] : 0u;  // real ~slots are > 0
    const unsigned ms = wave_max4_u32(es[0], es[1], es[2], es[3], lane);
    if (store && lane < 4) {
      out[tok * k + r] = cand_value(((cand_t)mo << 32) | ms);
      oslot[tok * k + r] = (int)~ms;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const unsigned mst = (unsigned)__builtin_amdgcn_readlane((int)ms, (t == 1) ? 2 : (t == 2) ? 1 : t);
      const bool take = o[t][0] == mot[t] && sl[t][0] == mst;  // drop the winner from its list
#pragma unroll
      for (int i = 0; i < 3; ++i) o[t][i] = take ? o[t][i + 1] : o[t][i], sl[t][i] = take ? sl[t][i + 1] : sl[t][i];
      o[t][3] = take ? NONE_O : o[t][3];
      sl[t][3] = take ? NONE_S : sl[t][3];
    }
  }
}

// wave_sum4's reduce-scatter for smooth pooling states: every lane ends with the wave's merged
// (m, s, t) of token wave_sum4_token(lane).  Merges are commutative bit for bit, and the two swap
// steps hand both lanes of a pair the same two operands, so the result does not depend on the lane.
template <int OP>
__device__ __forceinline__ void wave_merge4(const float (&m)[4], const float (&s)[4], const float (&t)[4], int lane,
                                            float p, int pint, float& mo, float& so, float& to) {
  const bool odd = lane & 1, hi = lane & 2;
  float m0 = odd ? m[2] : m[0], s0 = odd ? s[2] : s[0], t0 = odd ? t[2] : t[0];
  float m1 = odd ? m[3] : m[1], s1 = odd ? s[3] : s[1], t1 = odd ? t[3] : t[1];
  sm_merge<OP>(m0, s0, t0, dpp<0xB1>(odd ? m[0] : m[2]), dpp<0xB1>(odd ? s[0] : s[2]), dpp<0xB1>(odd ? t[0] : t[2]), p,
               pint);  // quad_perm(1,0,3,2)
  sm_merge<OP>(m1, s1, t1, dpp<0xB1>(odd ? m[1] : m[3]), dpp<0xB1>(odd ? s[1] : s[3]), dpp<0xB1>(odd ? t[1] : t[3]), p,
               pint);
  float cm = hi ? m1 : m0, cs = hi ? s1 : s0, ct = hi ? t1 : t0;
  sm_merge<OP>(cm, cs, ct, dpp<0x4E>(hi ? m0 : m1), dpp<0x4E>(hi ? s0 : s1), dpp<0x4E>(hi ? t0 : t1), p,
               pint);  // quad_perm(2,3,0,1)
  sm_merge<OP>(cm, cs, ct, dpp<0x124>(cm), dpp<0x124>(cs), dpp<0x124>(ct), p, pint);  // row_ror:4
  sm_merge<OP>(cm, cs, ct, dpp<0x128>(cm), dpp<0x128>(cs), dpp<0x128>(ct), p, pint);  // row_ror:8
  {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(cm), __float_as_uint(cm), false, false);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(cs), __float_as_uint(cs), false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(ct), __float_as_uint(ct), false, false);
    cm = __uint_as_float(a[0]), cs = __uint_as_float(b[0]), ct = __uint_as_float(c[0]);
    sm_merge<OP>(cm, cs, ct, __uint_as_float(a[1]), __uint_as_float(b[1]), __uint_as_float(c[1]), p, pint);
  }
  {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(cm), __float_as_uint(cm), false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(cs), __float_as_uint(cs), false, false);
    const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(ct), __float_as_uint(ct), false, false);
    cm = __uint_as_float(a[0]), cs = __uint_as_float(b[0]), ct = __uint_as_float(c[0]);
    sm_merge<OP>(cm, cs, ct, __uint_as_float(a[1]), __uint_as_float(b[1]), __uint_as_float(c[1]), p, pint);
  }
  mo = cm, so = cs, to = ct;
}

// Per token the lane's smooth state over its valid neurons (vmask bit j: neuron j valid) -- the
// largest u (or a), the sum of 2^(u - m) (or (a / m)^p) and, for softmax-weighted, of 2^(u - m) a --
// merged over the wave: every lane ends with the merged state of token wave_sum4_token(lane).
template <int OP, int NPL, int ACT = GL_ACT_RELU>
__device__ __forceinline__ void smooth_reduce(const float (&z)[NPL][4], unsigned vmask, int lane, float scale, float p,
                                              int pint, float& mo, float& so, float& to) {
  float m[4], s[4], t[4];
  const float ninf = -__builtin_inff();
#pragma unroll
  for (int tk = 0; tk < 4; ++tk) {
    if constexpr (OP == SM_POW) {
      float a[NPL], mx = 0.f;
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        a[j] = ((vmask >> j) & 1u) ? __builtin_fmaxf(z[j][tk], 0.f) : 0.f;
        mx = __builtin_fmaxf(mx, a[j]);
      }
      const float inv = mx > 0.f ? 1.f / mx : 0.f;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < NPL; ++j) acc += pow_p(a[j] * inv, p, pint);
      m[tk] = mx, s[tk] = acc, t[tk] = 0.f;
    } else {
      float a[NPL], u[NPL], mx = ninf;
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        const bool v = (vmask >> j) & 1u;
        const float aj = act_f<ACT>(z[j][tk]);
        a[j] = v ? aj : 0.f;
        u[j] = v ? aj * scale : ninf;
        mx = __builtin_fmaxf(mx, u[j]);
      }
      const float base = mx == ninf ? 0.f : mx;
      float acc = 0.f, acct = 0.f;
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        const float e = __builtin_amdgcn_exp2f(u[j] - base);
        acc += e;
        if constexpr (OP == SM_SW) acct = __builtin_fmaf(e, a[j], acct);
      }
      m[tk] = mx, s[tk] = acc, t[tk] = acct;
    }
  }
  wave_merge4<OP>(m, s, t, lane, p, pint, mo, so, to);
}

// Smooth pooling tile (LogMeanExp, power mean, softmax-weighted; pytorch_reference.py:80-100): z of
// the lane's neurons for the tile's 4 tokens, their states merged over the wave (smooth_reduce);
// lanes 0-3 store (m, s, t) per token.
template <int K, int NPL, int ACT, bool FAR, int OP, int PI = -1, int RA = (K == 8 ? 4 : 8), typename SRC = const char*>
__device__ __forceinline__ void fwd_tile_smooth(SRC xsb, const unsigned (&addr)[NPL][K], const float (&w)[NPL][K],
                                                const float (&bias)[NPL], unsigned vmask, float* out, bool store,
                                                int lane, float scale, float p, int pint) {
  float z[NPL][4];
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
    float z0 = bias[j], z1 = bias[j], z2 = bias[j], z3 = bias[j];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      z0 = __builtin_fmaf(xc[k].x, w[j][k], z0);
      z1 = __builtin_fmaf(xc[k].y, w[j][k], z1);
      z2 = __builtin_fmaf(xc[k].z, w[j][k], z2);
      z3 = __builtin_fmaf(xc[k].w, w[j][k], z3);
    }
    z[j][0] = z0, z[j][1] = z1, z[j][2] = z2, z[j][3] = z3;
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < NPL) {
#pragma unroll
      for (int k = 0; k < RA; ++k) xc[k] = xn[k];
    }
  }
  float mo, so, to;
  if constexpr (OP == SM_POW && PI > 0) {
    // a kernel of its own per integer p: its registers are those of that power alone
    smooth_reduce<OP, NPL>(z, vmask, lane, scale, p, PI, mo, so, to);
  } else if constexpr (OP == SM_POW) {
    // p as a literal where it is 1, 2, 4 or 8: the inlined powers then fold to products (with p
    // read at run time the branches of every power cost 63.5 against 33.0 ms per C2 forward)
    switch (pint) {
      case 1: smooth_reduce<OP, NPL>(z, vmask, lane, scale, p, 1, mo, so, to); break;
      case 2: smooth_reduce<OP, NPL>(z, vmask, lane, scale, p, 2, mo, so, to); break;
      case 4: smooth_reduce<OP, NPL>(z, vmask, lane, scale, p, 4, mo, so, to); break;
      case 8: smooth_reduce<OP, NPL>(z, vmask, lane, scale, p, 8, mo, so, to); break;
      default: smooth_reduce<OP, NPL>(z, vmask, lane, scale, p, 0, mo, so, to); break;
    }
  } else {
    smooth_reduce<OP, NPL, ACT>(z, vmask, lane, scale, p, pint, mo, so, to);
  }
  if (store && lane < 4) {
    float* o = out + wave_sum4_token(lane) * 3;
    o[0] = mo, o[1] = so, o[2] = to;
  }
}

// pool kinds of the forward tile
constexpr int PK_SUM = 0, PK_MAX = 1, PK_TOPK = 2, PK_LME = 3, PK_POW = 4, PK_SW = 5;
// the power mean with p = 1, 2, 4 or 8 as a literal: PK_POW_I + p (PK_POW: p read at run time)
constexpr int PK_POW_I = 8;
constexpr bool pk_smooth(int pk) { return pk >= PK_LME; }
constexpr int pk_pint(int pk) { return pk > PK_POW_I ? pk - PK_POW_I : -1; }
constexpr int pk_sm_op(int pk) { return pk == PK_LME ? SM_LME : (pk == PK_POW || pk_pint(pk) > 0 ? SM_POW : SM_SW); }

// sum / mean, max or top-k tile
template <int K, int NPL, int ACT, bool FAR, int PK, int TKW, typename SRC = const char*, typename MB = NoBits>
__device__ __forceinline__ void fwd_tile_any(SRC xsb, const unsigned (&addr)[NPL][K], const float (&w)[NPL][K],
                                             const float (&bias)[NPL], const int (&slot)[NPL], float* out, int* oslot,
                                             int k, bool store, int lane, MB& mb) {
  if constexpr (PK == PK_MAX) fwd_tile_max<K, NPL, ACT, FAR>(xsb, addr, w, bias, slot, out, oslot, store, lane);
  else if constexpr (PK == PK_TOPK)
    fwd_tile_topk<K, NPL, ACT, FAR, TKW>(xsb, addr, w, bias, slot, out, oslot, k, store, lane);
  else
    fwd_tile<K, NPL, ACT, FAR>(xsb, addr, w, bias, out, store, lane, mb);
}

// smooth pools: the tile needs the validity bits and the operator's parameters
template <int K, int NPL, int ACT, bool FAR, int PK, int TKW, typename SRC = const char*, typename MB = NoBits>
__device__ __forceinline__ void fwd_tile_dispatch(SRC xsb, const unsigned (&addr)[NPL][K], const float (&w)[NPL][K],
                                                  const float (&bias)[NPL], const int (&slot)[NPL], unsigned vmask,
                                                  float* out, int* oslot, int k, bool store, int lane, const FwdK& p,
                                                  MB& mb) {
  if constexpr (pk_smooth(PK))
    fwd_tile_smooth<K, NPL, ACT, FAR, pk_sm_op(PK), pk_pint(PK)>(xsb, addr, w, bias, vmask, out, store, lane, p.scale, p.pparam,
                                                    p.pint);
  else
    fwd_tile_any<K, NPL, ACT, FAR, PK, TKW>(xsb, addr, w, bias, slot, out, oslot, k, store, lane, mb);
}

template <int K, int NPL, int WAVES, int ACT, bool DBUF, bool WS = false, int PK = PK_SUM, bool XG = false,
          bool SMALL = false, int TB = BT, bool XB = false, bool FM = false>
// SMALL: two workgroups share a CU, so a wave must fit 128 VGPRs (4 waves per SIMD)
__global__ void __launch_bounds__(WAVES * 64, SMALL ? 16 / WAVES * WAVES / 4 : 1) fwd_kernel(FwdK p) {
  // WS: xa holds both stage regions (2 * WS_TILES * nsl <= 2 * XTILE_DB slots, XTILE_DB with
  // SMALL); XG: no LDS tile; SMALL: one single-buffered tile of at most XTILE_DB 16-byte slots, so
  // two workgroups share a CU.  TB: tokens per tile (4, or 2 for the two-token tiles of DBUF sum /
  // mean: D x 8 bytes per buffer)
  // XB: 4-token tiles of raw bf16 (8-byte slots, bf16 X), one buffer (SMALL) or two
  static_assert(TB == BT || (TB == 2 && DBUF && !WS && !XG && PK == PK_SUM), "two-token tiles: sum / mean, two buffers");
  static_assert(!XB || (TB == BT && (DBUF || SMALL || WS) && !XG && PK == PK_SUM), "bf16 tiles: sum / mean");
  static_assert(!FM || (TB == BT && PK == PK_SUM && ACT == GL_ACT_RELU), "ReLU bits: 4-token tiles, sum / mean");
  constexpr int SLOT = XB ? 8 : 4 * TB;  // bytes per input of a tile or stage
  __shared__ float4 xa[WS ? (SMALL ? XTILE_DB : 2 * XTILE_DB) : (XG ? 1 : (DBUF || SMALL ? XTILE_DB : XTILE_SB))];
  __shared__ float4 xb[DBUF ? XTILE_DB : 1];
  // top-k: the ranked tile's per-wave candidate lists, where the CU's LDS has room for them
  constexpr int TKW = PK == PK_TOPK && (SMALL ? 2 : 1) * (sizeof(xa) + sizeof(xb) + WAVES * 4 * TK_CAP * 8) <= 160 * 1024
                          ? WAVES
                          : 0;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar chunk addressing
  long long chunk = (long long)blockIdx.x * WAVES + wave;
  const bool active = chunk < p.n_chunks;
  if (!active) chunk = p.n_chunks - 1;  // idle waves of the last block recompute a real chunk, store nothing
  const long long g = chunk / p.cpg;
  const int s_lo = (int)(chunk % p.cpg) * 64 * NPL;
  const int ext = pool_ext((int)g, p.S, p.sps, p.gs);  // slots of the pool inside its group
  const int n_g = min(p.counts[g], ext);
  const long long nb = pool_base((int)g, p.S, p.sps, p.gs);  // the pool's first neuron

  unsigned addr[NPL][K];
  float w[NPL][K];
  float bias[NPL];
  int slot[NPL];  // max / top-k pooling: pool slot of each neuron
  unsigned vmask = 0u;  // smooth pools: bit j set when neuron j is a valid slot
  // window staging: this wave's pool is slot pk of the workgroup's staged pools, window start lo
  const int g_first = (int)((long long)blockIdx.x * WAVES / p.cpg);
  const int pk = WS ? (int)(g - g_first) : 0;
  const int lo = WS ? (int)__builtin_amdgcn_readfirstlane(p.win[g]) : 0;
  // the lane's neurons: input addresses, weights, bias, slots
  if constexpr (WS) {
    // pool windows: the parameter dtype tested per load (the set-up below, written as a generic
    // lambda, added spills to these kernels)
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      uint32_t order;
      const int s = sched_slot(p.sched, p.nwin, p.S, g, s_lo, j, lane, order);
      const bool valid = s < n_g;
      const long long n = nb + (s < ext ? s : ext - 1);  // in-bounds address; invalid slots masked
#pragma unroll
      for (int ks = 0; ks < K; ++ks) {
        const int k = sched_k<K>(order, ks);  // the pooled sum does not depend on the visiting order
        int d = rec_index(p.idx, n, k, K, p.rs);
        d = (d < 0 || !valid) ? 0 : (d >= p.D ? p.D - 1 : d);  // host validates; clamp keeps LDS reads in bounds
        addr[j][ks] = win_addr<SLOT>(d, pk, lo, p.ww);
        const float wl = ld_param(p.W, p.wbf, n * K + k);
        w[j][ks] = valid ? wl : 0.f;
      }
      const float bl = ld_param(p.bias, p.wbf, n);
      bias[j] = valid ? bl : ((PK == PK_MAX || PK == PK_TOPK) ? -__builtin_inff() : 0.f);
      slot[j] = s;
      vmask |= (unsigned)valid << j;
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
        const bool valid = s < n_g;
        const long long n = nb + (s < ext ? s : ext - 1);  // in-bounds address; invalid slots masked
#pragma unroll
        for (int ks = 0; ks < K; ++ks) {
          const int k = sched_k<K>(order, ks);  // the pooled sum does not depend on the visiting order
          int d = rec_index(p.idx, n, k, K, p.rs);
          d = (d < 0 || !valid) ? 0 : (d >= p.D ? p.D - 1 : d);  // host validates; clamp keeps LDS reads in bounds
          addr[j][ks] = (unsigned)d * SLOT;
          const float wl = ld_param_t<BF>(p.W, n * K + k);
          w[j][ks] = valid ? wl : 0.f;
        }
        const float bl = ld_param_t<BF>(p.bias, n);
        bias[j] = valid ? bl : ((PK == PK_MAX || PK == PK_TOPK) ? -__builtin_inff() : 0.f);
        slot[j] = s;
        vmask |= (unsigned)valid << j;
      }
    };
    if (p.wbf) setup(std::true_type{});
    else setup(std::false_type{});
  }

  // Token tiles reach LDS by LDS-DMA (dma_tile).  DBUF: tile t + 1 is loaded into the other
  // buffer while tile t is read, one barrier per tile; tiles alternate xa (even t) and xb (odd t),
  // each buffer read through its own array.  Otherwise: load, wait, read.  The copies are issued
  // from inline asm: a copy the compiler sees in flight during the gather makes it wait for all
  // LDS reads (lgkmcnt(0)) before each use instead of only the ones the use needs.
  constexpr int NT = WAVES * 64;
  const int kp = PK == PK_TOPK ? p.topk : (pk_smooth(PK) ? 3 : 1);  // floats per token: candidates or state
  float* out = p.part + chunk * p.b_pad * kp;
  int* oslot = (PK == PK_MAX || PK == PK_TOPK) ? p.pslot + chunk * p.b_pad * kp : nullptr;
  const bool store = active;
  // FM: every tile's ReLU bits go out as one 16-bit word per lane (128 contiguous bytes per wave)
  static_assert(!FM || NPL == 4, "16 bits per lane and tile");
  std::conditional_t<FM, ReluBits, NoBits> mb{};
  // the chunk's row of words as a scalar base; a tile's store adds a 32-bit offset
  char* const fmb = FM ? const_cast<char*>(uniform_ptr(p.fm + (chunk * p.fm_tiles + p.fm_t0) * 64)) : nullptr;
  auto bits_done = [&](int t) {
    if constexpr (FM) {
      if (store) *reinterpret_cast<uint16_t*>(fmb + ((unsigned)t * 128u + (unsigned)lane * 2u)) = (uint16_t)mb.bits;
      mb.bits = 0u;
    }
  };
  if constexpr (WS) {
    // window staging: WS_TILES tiles per stage and barrier; tile t at input (t mod 2 WS_TILES) * nsl
    // of the stage regions (IB bytes per input)
    const WinLayout L{p.win, p.ww, p.npw, g_first, p.G};
    const int nsl = p.npw * p.ww;
    const unsigned tstep = (unsigned)nsl * (unsigned)SLOT;
    const int rslots = WS_TILES * nsl * (int)SLOT / 16;  // 16-byte slots per region
    dma_window_stage<SLOT>(p.xt, xa, 0, p.n_tiles, p.D, L, WAVES);
    stage_wait();
    __syncthreads();
    for (int t0 = 0; t0 < p.n_tiles; t0 += WS_TILES) {
      const int r = (t0 / WS_TILES) & 1;
      // region r ^ 1 was last read in the previous stage, which every wave finished before the barrier
      if (t0 + WS_TILES < p.n_tiles)
        dma_window_stage<SLOT>(p.xt, xa + (r ^ 1) * rslots, t0 + WS_TILES, p.n_tiles, p.D, L, WAVES);
      const int tn = p.n_tiles - t0 < WS_TILES ? p.n_tiles - t0 : WS_TILES;
      for (int tt = 0; tt < tn; ++tt) {
        const int t = t0 + tt;
        if constexpr (XB)
          fwd_tile_bf4<K, NPL, ACT, false>(reinterpret_cast<const char*>(xa), addr, w, bias, out + t * BT, store, lane,
                                           mb);
        else
          fwd_tile_dispatch<K, NPL, ACT, false, PK, TKW>(reinterpret_cast<const char*>(xa), addr, w, bias, slot, vmask,
                                                    out + t * BT * kp, oslot + t * BT * kp, kp, store, lane, p, mb);
        bits_done(t);
        // next tile's slot; after the last tile of region 1 back to region 0
        const unsigned step = (t & (2 * WS_TILES - 1)) == 2 * WS_TILES - 1 ? tstep - 2u * WS_TILES * tstep : tstep;
#pragma unroll
        for (int j = 0; j < NPL; ++j)
#pragma unroll
          for (int k = 0; k < K; ++k) addr[j][k] += step;
      }
      stage_wait();
      __syncthreads();
    }
  } else if constexpr (XG) {
    // D too wide for an LDS tile: the lanes gather their 16-byte slots straight from the token tile
    // in global memory with buffer loads (D x 16 bytes, L2-resident while the workgroups of the
    // launch read it), with no staging and no barriers
    for (int t = 0; t < p.n_tiles; ++t) {
      fwd_tile_dispatch<K, NPL, ACT, false, PK, TKW>(xbuf(p.xt + (long long)t * p.D, p.D), addr, w, bias, slot, vmask,
                                                out + t * BT * kp, oslot + t * BT * kp, kp, store, lane, p, mb);
      bits_done(t);
    }
  } else if constexpr (DBUF) {
    const int ns = (int)((long long)p.D * SLOT / 16);  // 16-byte slots per tile
    dma_tile(p.xt, xa, ns, NT);
    for (int t = 0; t < p.n_tiles; t += 2) {
      stage_wait();
      __syncthreads();  // tile t is in xa; every wave is done with xb (tile t - 1)
      if (t + 1 < p.n_tiles) dma_tile(p.xt + (long long)(t + 1) * ns, xb, ns, NT);
      if constexpr (XB)
        fwd_tile_bf4<K, NPL, ACT, false>(reinterpret_cast<const char*>(xa), addr, w, bias, out + t * BT, store, lane,
                                         mb);
      else if constexpr (TB == 2)
        fwd_tile2<K, NPL, ACT, false>(reinterpret_cast<const char*>(xa), addr, w, bias, out + t * 2, store, lane);
      else
        fwd_tile_dispatch<K, NPL, ACT, false, PK, TKW>(reinterpret_cast<const char*>(xa), addr, w, bias, slot, vmask,
                                                  out + t * BT * kp, oslot + t * BT * kp, kp, store, lane, p, mb);
      bits_done(t);
      if (t + 1 < p.n_tiles) {
        stage_wait();
        __syncthreads();  // tile t + 1 is in xb; every wave is done with xa
        if (t + 2 < p.n_tiles) dma_tile(p.xt + (long long)(t + 2) * ns, xa, ns, NT);
        if constexpr (XB)
          fwd_tile_bf4<K, NPL, ACT, true>(reinterpret_cast<const char*>(xb), addr, w, bias, out + (t + 1) * BT, store,
                                          lane, mb);
        else if constexpr (TB == 2)
          fwd_tile2<K, NPL, ACT, true>(reinterpret_cast<const char*>(xb), addr, w, bias, out + (t + 1) * 2, store, lane);
        else
          fwd_tile_dispatch<K, NPL, ACT, true, PK, TKW>(reinterpret_cast<const char*>(xb), addr, w, bias, slot, vmask,
                                                   out + (t + 1) * BT * kp, oslot + (t + 1) * BT * kp, kp, store, lane, p,
                                                   mb);
        bits_done(t + 1);
      }
    }
  } else {
    const int ns = (int)((long long)p.D * SLOT / 16);  // 16-byte slots per tile
    for (int t = 0; t < p.n_tiles; ++t) {
      __syncthreads();  // every wave is done with tile t - 1
      dma_tile(p.xt + (long long)t * ns, xa, ns, NT);
      stage_wait();
      __syncthreads();
      if constexpr (XB)
        fwd_tile_bf4<K, NPL, ACT, false>(reinterpret_cast<const char*>(xa), addr, w, bias, out + t * BT, store, lane,
                                         mb);
      else
        fwd_tile_dispatch<K, NPL, ACT, false, PK, TKW>(reinterpret_cast<const char*>(xa), addr, w, bias, slot, vmask,
                                                  out + t * BT * kp, oslot + t * BT * kp, kp, store, lane, p, mb);
      bits_done(t);
    }
  }
}

// pre[b, g] = scale_g * sum_{c < cpg} part[g*cpg + c, b]  (fixed order, c ascending), transposed to
// [B, G] through LDS.  A thread sums 4 adjacent tokens of one pool with 16-byte loads, 8 chunk
// rows in flight (the add order per element is unchanged); 32 pools x 32 tokens per workgroup.
__global__ void __launch_bounds__(256) fwd_finalize_kernel(const float* __restrict__ part, const int32_t* __restrict__ counts,
                                                           float* __restrict__ pre, int B, int G, int cpg, int b_pad,
                                                           int b0, int pool) {
  __shared__ float tile[32][33];  // [token][pool]
  const int g0 = blockIdx.x * 32, bb0 = blockIdx.y * 32;
  const int gl = threadIdx.x >> 3, q4 = (threadIdx.x & 7) * 4;  // pool g0 + gl, tokens bb0 + q4 .. + 3
  const int g = g0 + gl;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (g < G && bb0 + q4 < b_pad) {  // b_pad is a multiple of 4: the 4 tokens lie inside the rows
    const float4* src = reinterpret_cast<const float4*>(part + (long long)g * cpg * b_pad + bb0 + q4);
    const long long cs = b_pad / 4;  // float4 stride between a pool's chunk rows
    int c = 0;
    for (; c + 8 <= cpg; c += 8) {
      float4 t[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) t[i] = src[(c + i) * cs];
#pragma unroll
      for (int i = 0; i < 8; ++i) v.x += t[i].x, v.y += t[i].y, v.z += t[i].z, v.w += t[i].w;
    }
    for (; c < cpg; ++c) {
      const float4 t = src[c * cs];
      v.x += t.x, v.y += t.y, v.z += t.z, v.w += t.w;
    }
    if (pool == GL_POOL_MEAN) {
      const float n = (float)counts[g];
      v.x = v.x / n, v.y = v.y / n, v.z = v.z / n, v.w = v.w / n;
    }
  }
  tile[q4][gl] = v.x, tile[q4 + 1][gl] = v.y, tile[q4 + 2][gl] = v.z, tile[q4 + 3][gl] = v.w;
  __syncthreads();
  for (int r = threadIdx.x >> 5; r < 32; r += 8) {
    const int b = bb0 + r, gg = g0 + (threadIdx.x & 31);
    if (gg < G && b0 + b < B && b < b_pad) pre[(long long)(b0 + b) * G + gg] = tile[r][threadIdx.x & 31];
  }
}

// Max pooling: pre[b, g] = the largest partial maximum over the pool's cpg chunks, winner[b, g] its
// slot (the smaller slot on ties, as merge_finalize, kernels/ops.py:189-195); tiled transpose.
__global__ void __launch_bounds__(256) fwd_finalize_max_kernel(const float* __restrict__ part, const int* __restrict__ pslot,
                                                               float* __restrict__ pre, int32_t* __restrict__ winner, int B,
                                                               int G, int cpg, int b_pad) {
  __shared__ float tile[32][33];
  __shared__ int tslot[32][33];
  const int g0 = blockIdx.x * 32, bb0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int r = ty; r < 32; r += 8) {
    const int g = g0 + r, b = bb0 + tx;
    float m = -__builtin_inff();
    int sl = 0x7fffffff;
    if (g < G && b < b_pad) {
      const long long o = (long long)g * cpg * b_pad + b;
      for (int c = 0; c < cpg; ++c) vmax_pair(m, sl, part[o + (long long)c * b_pad], pslot[o + (long long)c * b_pad]);
    }
    tile[r][tx] = m;
    tslot[r][tx] = sl;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int b = bb0 + r, g = g0 + tx;
    if (g < G && b < B && b < b_pad) {
      pre[(long long)b * G + g] = tile[tx][r];
      if (winner) winner[(long long)b * G + g] = tslot[tx][r];
    }
  }
}

// Top-k mean pooling: the k largest raw z over the pool's cpg chunk lists (each sorted best first,
// k long), ties to the smaller slot (the reference's stable descending sort); pre[b, g] = the mean
// of act(z) over the first kk = min(n_g, k) of them, topk_slot[b, g, j] their slots (-1 past kk).
// One thread per (token, pool) merges the lists (at most FWD_TOPK_CPG of them); consecutive threads
// take consecutive tokens, so each candidate load of a wave reads 64 adjacent k-entry rows.
constexpr int FWD_TOPK_CPG = 16;

template <int ACT>
__global__ void __launch_bounds__(256) fwd_finalize_topk_kernel(const float* __restrict__ part, const int* __restrict__ pslot,
                                                                const int32_t* __restrict__ counts, float* __restrict__ pre,
                                                                int32_t* __restrict__ topk_slot, int B, int G, int cpg,
                                                                int b_pad, int k) {
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long long)B * G) return;
  const int b = (int)(t % B), g = (int)(t / B);
  const long long i = (long long)b * G + g;  // [B, G] output element
  int ptr[FWD_TOPK_CPG];
#pragma unroll
  for (int c = 0; c < FWD_TOPK_CPG; ++c) ptr[c] = 0;
  const int n_g = counts[g];
  const int kk = n_g < k ? n_g : k;
  float sum = 0.f;
  for (int j = 0; j < kk; ++j) {
    int best = -1;
    float bv = 0.f;
    int bs = 0;
#pragma unroll
    for (int c = 0; c < FWD_TOPK_CPG; ++c) {
      if (c < cpg && ptr[c] < k) {
        const long long o = (((long long)g * cpg + c) * b_pad + b) * k + ptr[c];
        const float v = part[o];
        const int sl = pslot[o];
        if (best < 0 || cand_key(v, ~(unsigned)sl) > cand_key(bv, ~(unsigned)bs)) best = c, bv = v, bs = sl;
      }
    }
#pragma unroll
    for (int c = 0; c < FWD_TOPK_CPG; ++c) ptr[c] += c == best;
    sum += act_f<ACT>(bv);
    if (topk_slot) topk_slot[i * k + j] = bs;
  }
  if (topk_slot)
    for (int j = kk; j < k; ++j) topk_slot[i * k + j] = -1;
  pre[i] = sum / (float)kk;
}

// k = 8 with at most 4 chunks per pool (pools of up to 1024 slots): the same merge with the lists
// in registers.  Every thread loads its 4 lists with 16-byte loads (the lanes of a wave read
// consecutive tokens' lists, 2 KiB in a row) instead of re-reading every head per pick, and
// writes its 8 slots with two 16-byte stores.  Picks and summation order are those of
// fwd_finalize_topk_kernel, so the results are bit-identical.
constexpr int FWD_TOP8_CPG = 4;

template <int ACT>
__global__ void __launch_bounds__(256) fwd_finalize_top8_kernel(const float* __restrict__ part, const int* __restrict__ pslot,
                                                                const int32_t* __restrict__ counts, float* __restrict__ pre,
                                                                int32_t* __restrict__ topk_slot, int B, int G, int cpg,
                                                                int b_pad) {
  constexpr int KP = 8, CP = FWD_TOP8_CPG;
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long long)B * G) return;
  const int b = (int)(t % B), g = (int)(t / B);
  const long long i = (long long)b * G + g;
  float v[CP][KP];
  int s[CP][KP];
#pragma unroll
  for (int c = 0; c < CP; ++c) {
    if (c < cpg) {
      const long long o = (((long long)g * cpg + c) * b_pad + b) * KP;
      const float4 a0 = *reinterpret_cast<const float4*>(part + o), a1 = *reinterpret_cast<const float4*>(part + o + 4);
      const int4 q0 = *reinterpret_cast<const int4*>(pslot + o), q1 = *reinterpret_cast<const int4*>(pslot + o + 4);
      v[c][0] = a0.x, v[c][1] = a0.y, v[c][2] = a0.z, v[c][3] = a0.w;
      v[c][4] = a1.x, v[c][5] = a1.y, v[c][6] = a1.z, v[c][7] = a1.w;
      s[c][0] = q0.x, s[c][1] = q0.y, s[c][2] = q0.z, s[c][3] = q0.w;
      s[c][4] = q1.x, s[c][5] = q1.y, s[c][6] = q1.z, s[c][7] = q1.w;
    } else {
#pragma unroll
      for (int e = 0; e < KP; ++e) v[c][e] = -__builtin_inff(), s[c][e] = 0x7fffffff;
    }
  }
  const int n_g = counts[g];
  const int kk = n_g < KP ? n_g : KP;
  float sum = 0.f;
  int out[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    int bc = 0;
    float bv = v[0][0];
    int bs = s[0][0];
#pragma unroll
    for (int c = 1; c < CP; ++c) {
      const bool tk = cand_key(v[c][0], ~(unsigned)s[c][0]) > cand_key(bv, ~(unsigned)bs);
      bc = tk ? c : bc, bv = tk ? v[c][0] : bv, bs = tk ? s[c][0] : bs;
    }
    out[j] = j < kk ? bs : -1;
    if (j < kk) sum += act_f<ACT>(bv);
    // drop the head of the list it came from; after j + 1 picks a list is read at most up to
    // position KP - 2 - j, and a list popped p <= j times still holds valid entries to KP - 1 - p
#pragma unroll
    for (int c = 0; c < CP; ++c) {
      const bool take = c == bc;
#pragma unroll
      for (int e = 0; e + 1 < KP - j; ++e) v[c][e] = take ? v[c][e + 1] : v[c][e], s[c][e] = take ? s[c][e + 1] : s[c][e];
    }
  }
  if (topk_slot) {
    *reinterpret_cast<int4*>(topk_slot + i * KP) = make_int4(out[0], out[1], out[2], out[3]);
    *reinterpret_cast<int4*>(topk_slot + i * KP + 4) = make_int4(out[4], out[5], out[6], out[7]);
  }
  pre[i] = sum / (float)kk;
}

// Smooth pools: merge the pool's cpg chunk states in a fixed order, then pre and L2 = m + log2 s
// (kernels/ops.py:201-219): LogMeanExp pre = (L2 - log2 n_g) / scale, softmax-weighted pre = t / s,
// power mean pre = m (s / n_g)^(1/p) (0 when every activation is 0).  One thread per (token, pool).
template <int OP>
__global__ void __launch_bounds__(256) fwd_finalize_smooth_kernel(const float* __restrict__ part,
                                                                  const int32_t* __restrict__ counts, float* __restrict__ pre,
                                                                  float* __restrict__ lse, int B, int G, int cpg, int b_pad,
                                                                  float scale, float p, int pint) {
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long long)B * G) return;
  const int b = (int)(t % B), g = (int)(t / B);
  const float* q = part + ((long long)g * cpg * b_pad + b) * 3;
  float m = q[0], sv = q[1], tv = q[2];
  for (int c = 1; c < cpg; ++c) {
    const float* r = q + (long long)c * b_pad * 3;
    sm_merge<OP>(m, sv, tv, r[0], r[1], r[2], p, pint);
  }
  const float n = (float)counts[g];
  const long long i = (long long)b * G + g;
  if constexpr (OP == SM_POW) {
    float v = 0.f;
    if (m > 0.f) v = pint == 1 ? m * (sv / n) : m * __builtin_amdgcn_exp2f(__builtin_amdgcn_logf(sv / n) / p);
    pre[i] = v;
    if (lse) lse[i] = 0.f;
  } else {
    const float L2 = m + __builtin_amdgcn_logf(sv);
    pre[i] = OP == SM_LME ? (L2 - __builtin_amdgcn_logf(n)) / scale : tv / sv;
    if (lse) lse[i] = L2;
  }
}

// ---- host side -------------------------------------------------------------------------------
// 4 neurons per lane; 16 waves per workgroup at K = 8 (4 waves per SIMD, 128 VGPRs), 8 at K = 16
// (2 per SIMD: the parameters of 4 neurons of fan-in 16 take twice the registers).  Max pooling
// keeps a slot per neuron and a (value, slot) pair per token: 12 waves at K = 8, 4 at K = 16;
// top-k keeps a sorted list of 4 keys per token: 12 waves at K = 8 with the ranked tile (158 VGPRs,
// 16-key blocks; 32-key blocks took 190 VGPRs, 2 waves per SIMD: C2 top-8 forward 54.0 ms against
// 65.5 ms at 8 waves and 16-key blocks), 8 where the tile is single-buffered (the rounds spill 176
// bytes at 12), 4 at K = 16.
constexpr int FWD_NPL = 4;
static_assert(FWD_NPL == RELU_MASK_NPL, "the forward writes the ReLU bits chunk by chunk");
constexpr int fwd_waves(int K, int pk = PK_SUM, int act = GL_ACT_RELU) {
  // LogMeanExp and softmax-weighted at fan-in 8 with ReLU or identity neurons: 12 waves (3 per SIMD,
  // 130-136 VGPRs; C2 LogMeanExp forward 31.4 -> 26.2 ms against 8); the power mean (168 VGPRs
  // would spill 140-176 bytes per lane) and GELU neurons keep 8
  // the power mean with p = 1, 2 or 4 as a literal: 129-134 VGPRs at 12 waves (p = 8 and p read at
  // run time spill 88-176 bytes per lane)
  const bool sm12 = K == 8 && (pk == PK_LME || pk == PK_SW || (pk_pint(pk) > 0 && pk_pint(pk) < 8)) &&
                    act != GL_ACT_GELU;
  return K == 8 ? (pk == PK_SUM ? 16 : (pk == PK_MAX || pk == PK_TOPK || sm12 ? 12 : 8)) : (pk == PK_SUM ? 8 : 4);
}
static int pool_kind(int pool) {
  switch (pool) {
    case GL_POOL_MAX: return PK_MAX;
    case GL_POOL_TOPK_MEAN: return PK_TOPK;
    case GL_POOL_LME: return PK_LME;
    case GL_POOL_POWER: return PK_POW;
    case GL_POOL_SOFTMAX: return PK_SW;
    default: return PK_SUM;
  }
}
static bool pool_smooth(int pool) { return pool == GL_POOL_LME || pool == GL_POOL_POWER || pool == GL_POOL_SOFTMAX; }
static int smooth_pint(int pool, float param);
// the forward kernel's pool kind: the power mean's integer p is part of it
static int fwd_pool_kind(const GlFwdArgs* a) {
  const int pi = smooth_pint(a->pool, a->pool_param);
  return a->pool == GL_POOL_POWER && pi > 0 ? PK_POW_I + pi : pool_kind(a->pool);
}

// smooth pools: u = a * scale with scale = log2(e) / tau (LogMeanExp) or log2(e) * beta (softmax-weighted),
// the exact-product power for p in {1, 2, 4, 8}
static float smooth_scale(int pool, float param) {
  const float log2e = 1.4426950408889634f;
  return pool == GL_POOL_LME ? log2e / param : (pool == GL_POOL_SOFTMAX ? log2e * param : 1.f);
}
static int smooth_pint(int pool, float param) {
  if (pool != GL_POOL_POWER) return 0;
  return (param == 1.f || param == 2.f || param == 4.f || param == 8.f) ? (int)param : 0;
}

// Forward plan: the forward runs over token chunks of bf tokens (a multiple of BT) whose per-chunk
// partials (part_bytes + slot_bytes) fit the caller's part budget; every pass reloads the chunk
// parameters once and streams its own token tiles.  The per-token results do not depend on the
// chunking (same waves, same order), so any budget gives the same bits.  The default 8 GiB runs
// C2's top-8 mean in one pass of 256 tokens (67.2 ms) where 4 GiB took two (2 x 34.4 ms).
constexpr size_t FWD_PART_BUDGET_DEFAULT = 8ull << 30;

struct FwdPlan {
  int npl, waves, cpg, bf, n_passes;
  long long n_chunks;
  size_t xt_bytes, part_bytes, slot_bytes;
};

// bytes of partial results (values, plus slots for max / top-k) one token of a pass holds
static long long fwd_part_per_token(const GlFwdArgs* a, long long n_chunks) {
  // candidates per chunk and token (top-k), a smooth pool's (m, s, t) state, else one partial sum
  const long long kp = a->pool == GL_POOL_TOPK_MEAN ? a->topk : (pool_smooth(a->pool) ? 3 : 1);
  const bool sel = a->pool == GL_POOL_MAX || a->pool == GL_POOL_TOPK_MEAN;
  return n_chunks * kp * 4 * (sel ? 2 : 1);
}

// plan with token chunks of at most bf_cap tokens (<= 0: no cap beyond the part budget)
static FwdPlan fwd_plan(const GlFwdArgs* a, long long bf_cap = 0) {
  FwdPlan q;
  q.npl = FWD_NPL;
  q.waves = fwd_waves(a->K, fwd_pool_kind(a), a->act);
  q.cpg = ceil_div(a->S, 64 * q.npl);
  q.n_chunks = (long long)a->G * q.cpg;
  const long long kp = a->pool == GL_POOL_TOPK_MEAN ? a->topk : (pool_smooth(a->pool) ? 3 : 1);
  const bool sel = a->pool == GL_POOL_MAX || a->pool == GL_POOL_TOPK_MEAN;
  const long long per_token = fwd_part_per_token(a, q.n_chunks);
  const size_t budget = a->part_budget ? a->part_budget : FWD_PART_BUDGET_DEFAULT;
  const long long b_all = round_up(a->B, BT);
  long long bf = (long long)(budget / (size_t)per_token) / BT * BT;
  if (bf < BT) bf = BT;
  if (bf_cap > 0 && bf > bf_cap) bf = bf_cap;
  if (bf > b_all) bf = b_all;
  q.bf = (int)bf;
  q.n_passes = ceil_div(a->B, q.bf);
  q.xt_bytes = (size_t)round_up((long long)q.bf * a->D * 4, 256);
  q.part_bytes = (size_t)round_up(q.n_chunks * q.bf * kp * 4, 256);
  q.slot_bytes = sel ? q.part_bytes : 0;  // candidate slots
  return q;
}

template <int K, int NPL, int WAVES, int ACT, bool DBUF, bool WS, int PK, bool XG = false, bool SMALL = false,
          int TB = BT, bool XB = false>
static int launch_fwd(const FwdK& k, hipStream_t s) {
  auto fn = fwd_kernel<K, NPL, WAVES, ACT, DBUF, WS, PK, XG, SMALL, TB, XB>;
  if constexpr (PK == PK_SUM && ACT == GL_ACT_RELU && K == 8 && TB == BT)
    if (k.fm) fn = fwd_kernel<K, NPL, WAVES, ACT, DBUF, WS, PK, XG, SMALL, TB, XB, true>;
  dim3 grid((unsigned)ceil_div(k.n_chunks, WAVES));
  GL_LAUNCH(WS ? GL_KERNEL_FWD_WIN : GL_KERNEL_FWD, fn, grid, dim3(WAVES * 64), 0, s, k);
  GL_CHECK_LAUNCH();
  return 0;
}

// pool windows when they fit, else (D > XTILE_SB) gathers from the tiles in global memory, else
// tiles in LDS: one per workgroup with two workgroups per CU, or two buffers or one in a single
// workgroup per CU
template <int ACT, int K, int PK>
static int launch_fwd_buf(int D, const FwdK& k, hipStream_t s) {
  constexpr int W = fwd_waves(K, PK, ACT);
  if (k.win) {
    if (k.xb) {  // bf16 windows (sum / mean)
      if constexpr (PK == PK_SUM && W % 8 == 0)
        return k.ws_small ? launch_fwd<K, FWD_NPL, W / 2, ACT, false, true, PK, false, true, BT, true>(k, s)
                          : launch_fwd<K, FWD_NPL, W, ACT, false, true, PK, false, false, BT, true>(k, s);
      return GL_ERR_UNSUPPORTED;
    }
    if constexpr (W % 8 == 0 && !pk_smooth(PK))
      if (k.ws_small) return launch_fwd<K, FWD_NPL, W / 2, ACT, false, true, PK, false, true>(k, s);
    return launch_fwd<K, FWD_NPL, W, ACT, false, true, PK>(k, s);
  }
  // 8-byte-slot tiles (sum / mean, the host chose the format):
  // - bf16 X (even D <= 2 XTILE_DB): 4-token tiles of raw bf16 (64 KiB at D = 8192), one per
  //   workgroup and two workgroups per CU (C4 forward 81.8 -> 51.5 ms; two buffers in one
  //   workgroup: 56.3 ms);
  // - fp32 X, XTILE_DB < D <= 2 XTILE_DB: two-token tiles, two 64-KiB buffers in one workgroup of W waves (at C4, 81.7 ms
  //   against 83.7 ms for two workgroups of W / 2 waves with one tile each: the copy of the next
  //   tile overlaps the gathers, and the tile is shared by twice the neurons)
  if (k.xb || k.tb == 2) {
    if constexpr (PK == PK_SUM && W % 8 == 0) {
      if (k.xb) return launch_fwd<K, FWD_NPL, W / 2, ACT, false, false, PK, false, true, BT, true>(k, s);
      return launch_fwd<K, FWD_NPL, W, ACT, true, false, PK, false, false, 2>(k, s);
    }
    return GL_ERR_UNSUPPORTED;
  }
  if (D > XTILE_SB) return launch_fwd<K, FWD_NPL, W, ACT, false, false, PK, true>(k, s);
  // D <= XTILE_DB: two workgroups of W / 2 waves per CU, each with one 64-KiB tile, when W / 2 waves
  // spread evenly over the 4 SIMDs: while one workgroup waits at its tile barrier for its slowest
  // wave, the other computes (12% faster than one workgroup of W waves with two buffers for sum /
  // mean and top-k at C2; the smooth pools measured even)
  if constexpr (W % 8 == 0 && !pk_smooth(PK))
    if (D <= XTILE_DB) return launch_fwd<K, FWD_NPL, W / 2, ACT, false, false, PK, false, true>(k, s);
  // top-k over one single-buffered tile: no LDS left for the ranked tile's lists, and the rounds
  // spill at 12 waves
  constexpr int W1 = PK == PK_TOPK && K == 8 ? 8 : W;
  return D <= XTILE_DB ? launch_fwd<K, FWD_NPL, W, ACT, true, false, PK>(k, s)
                       : launch_fwd<K, FWD_NPL, W1, ACT, false, false, PK>(k, s);
}

template <int ACT, int PK>
static int launch_fwd_act(int K, int D, const FwdK& k, hipStream_t s) {
  return K == 8 ? launch_fwd_buf<ACT, 8, PK>(D, k, s) : launch_fwd_buf<ACT, 16, PK>(D, k, s);
}

template <int PK>
static int launch_fwd_any(int act, int K, int D, const FwdK& k, hipStream_t s) {
  if constexpr (pk_pint(PK) > 0) {
    return launch_fwd_act<GL_ACT_RELU, PK>(K, D, k, s);  // the power mean is ReLU only
  } else {
    if (act == GL_ACT_GELU) return launch_fwd_act<GL_ACT_GELU, PK>(K, D, k, s);
    return act == GL_ACT_RELU ? launch_fwd_act<GL_ACT_RELU, PK>(K, D, k, s) : launch_fwd_act<GL_ACT_IDENTITY, PK>(K, D, k, s);
  }
}

// Window staging applies when the staged windows of a workgroup's pools (npw of them, each ww
// inputs) fit a stage tile (<= WS_SLOTS) and are narrower than the full input width.
bool window_staging(const uint32_t* win, int width, int D, int waves, int cpg, int G, int* ww, int* npw,
                    int max_slots, int in_bytes) {
  if (!win || width < 1) return false;
  // 8-byte inputs: a staged window starts at the even input at or below the pool's first, one more
  const int w = (int)round_up(in_bytes == 8 ? width + 1 : width, 64);
  // pools spanned by `waves` consecutive chunks (cpg chunks per pool)
  int n = waves % cpg == 0 ? waves / cpg : (waves - 1) / cpg + 2;
  if (n > G) n = G;
  if ((long long)n * w * in_bytes > (long long)max_slots * 16 || (long long)n * w >= D) return false;
  *ww = w;
  *npw = n;
  return true;
}

int check_layer(int B, int D, int G, int S, int K, int act, int pool, const void* X, const int32_t* idx, const void* W,
                const void* bias, const int32_t* counts, int x_dtype, int w_dtype) {
  if (!X || !idx || !W || !bias || !counts) return GL_ERR_ARG;
  if (w_dtype != GL_DTYPE_F32 && w_dtype != GL_DTYPE_BF16) return GL_ERR_UNSUPPORTED;
  if (((uintptr_t)W & 3) != 0) return GL_ERR_ARG;  // the dX kernels read bf16 weights as 32-bit words
  if (B < 1 || D < 1 || G < 1 || S < 1) return GL_ERR_ARG;
  if (K != 8 && K != 16) return GL_ERR_UNSUPPORTED;
  if (act != GL_ACT_IDENTITY && act != GL_ACT_RELU && act != GL_ACT_GELU) return GL_ERR_UNSUPPORTED;
  if (pool < GL_POOL_MEAN || pool > GL_POOL_SOFTMAX) return GL_ERR_UNSUPPORTED;
  if (x_dtype != GL_DTYPE_F32 && x_dtype != GL_DTYPE_BF16) return GL_ERR_UNSUPPORTED;
  if ((long long)G * S > (1LL << 31) / 16) return GL_ERR_UNSUPPORTED;
  if (D > GL_MAX_INPUTS) return GL_ERR_UNSUPPORTED;  // wider tiles gather from global memory (XG kernels)
  return 0;
}

// smooth pools: temperature / beta > 0, p >= 1 with relu activations (the reference's LevelSpec
// checks, sparse_pooling/config.py:120-127)
int check_smooth(int pool, float param, int act) {
  if (pool == GL_POOL_LME || pool == GL_POOL_SOFTMAX) return param > 0.f && param < 3.0e38f ? 0 : GL_ERR_ARG;
  if (pool == GL_POOL_POWER) return (param >= 1.f && param < 3.0e38f && act == GL_ACT_RELU) ? 0 : GL_ERR_ARG;
  return 0;
}

int check_rec_shift(int rec_shift, int S, const void* sched) {
  if (rec_shift < 0 || rec_shift > 4) return GL_ERR_ARG;
  if (rec_shift > 0 && (S % (1 << rec_shift) != 0 || sched != nullptr)) return GL_ERR_ARG;
  return 0;
}

int check_geometry(int G, int S, int32_t* sps, int32_t* gs) {
  if (*sps < 0) return GL_ERR_ARG;
  if (*sps <= 1) {  // pools are groups: a group stride, if given, must be the pool size
    if (*gs != 0 && *gs != S) return GL_ERR_ARG;
    *sps = 1;
    *gs = S;
    return 0;
  }
  if (G % *sps != 0 || (long long)(*sps - 1) * S >= *gs || *gs > (long long)*sps * S) return GL_ERR_ARG;
  return 0;
}

// top-k mean: k a power of two in [1, 64] (the reference's LevelSpec check) and pools that the
// finalize's merge covers (cpg <= FWD_TOPK_CPG chunks of 256 slots)
int check_topk(int pool, int topk, int S) {
  if (pool != GL_POOL_TOPK_MEAN) return 0;
  if (topk < 1 || topk > 64 || (topk & (topk - 1)) != 0) return GL_ERR_ARG;
  if (ceil_div(S, 64 * FWD_NPL) > FWD_TOPK_CPG) return GL_ERR_UNSUPPORTED;
  return 0;
}

// The forward passes over token chunks of q.bf tokens with the workspace at ws (q's layout).
static int fwd_run(const GlFwdArgs* a, void* ws, const FwdPlan& q, hipStream_t s) {
  float4* xt = (float4*)ws;
  float* part = (float*)((char*)ws + q.xt_bytes);
  int* pslot = q.slot_bytes ? (int*)((char*)ws + q.xt_bytes + q.part_bytes) : nullptr;
  const int kpe = a->pool == GL_POOL_TOPK_MEAN ? a->topk : 1;
  for (int b0 = 0; b0 < a->B; b0 += q.bf) {
    // one pass: tokens [b0, b0 + Bc), written to rows b0.. of pre / winner
    const int Bc = a->B - b0 < q.bf ? a->B - b0 : q.bf;
    const int b_pad = (int)round_up(Bc, BT);
    float* pre = a->pre + (long long)b0 * a->G;
    int32_t* winner = a->winner ? a->winner + (long long)b0 * a->G * kpe : nullptr;
    FwdK k{xt, a->idx, (const float*)a->W, (const float*)a->bias, a->counts, part, pslot, kpe, a->sched, nullptr, q.n_chunks, a->D, a->S, q.cpg,
           b_pad / BT, b_pad, ceil_div(a->S, SCHED_WIN), a->G, 0, 0, a->rec_shift,
           smooth_scale(a->pool, a->pool_param), a->pool_param, smooth_pint(a->pool, a->pool_param)};
    k.sps = a->sps > 1 ? a->sps : 1;
    k.gs = a->sps > 1 ? a->gs : a->S;
    k.wbf = a->w_dtype == GL_DTYPE_BF16;
    if (a->relu_mask) {
      k.fm = (uint16_t*)a->relu_mask;
      k.fm_tiles = ceil_div(a->B, BT);
      k.fm_t0 = b0 / BT;
    }
    // sum / mean with bf16 X (even D <= 2 XTILE_DB) keeps X's bf16 values, 4 tokens per 8-byte slot,
    // in full tiles or windows: half the LDS bytes per gathered token for one exact widening per
    // value (C4 forward 81.8 -> 51.5 ms; at D = 4096 full tiles 16.4 -> 14.4 ms)
    k.xb = pool_kind(a->pool) == PK_SUM && a->x_dtype == GL_DTYPE_BF16 && a->D % 2 == 0 && a->D <= 2 * XTILE_DB;
    const int ib = k.xb ? 8 : 16;  // bytes per staged input
    // window staging: two workgroups of half the waves per CU when their windows fit half the slots
    // (the rule of the full-tile kernels: wave counts that spread evenly, not the smooth pools)
    if (q.waves % 8 == 0 && !pool_smooth(a->pool) &&
        window_staging(a->win, a->win_width, a->D, q.waves / 2, q.cpg, a->G, &k.ww, &k.npw, WS_SLOTS / 2, ib)) {
      k.win = a->win;
      k.ws_small = 1;
    } else if (window_staging(a->win, a->win_width, a->D, q.waves, q.cpg, a->G, &k.ww, &k.npw, WS_SLOTS, ib)) {
      k.win = a->win;
    }
    // fp32 X, sum / mean over full tiles of 4097..8192 inputs: two-token tiles (8-byte slots)
    k.tb = !k.xb && pool_kind(a->pool) == PK_SUM && !k.win && tiles_of_two(a->D) ? 2 : BT;
    k.n_tiles = b_pad / k.tb;
    if (k.xb)
      GL_TRY(launch_tile_x_bf16x4(a->X, a->sxb, a->B, a->D, b0, k.n_tiles, xt, s));
    else
      GL_TRY(launch_tile_x(a->X, a->sxb, a->x_dtype, a->B, a->D, b0, k.n_tiles, xt, s, k.tb));
    dim3 grid((unsigned)ceil_div(a->G, 32), (unsigned)ceil_div(b_pad, 32));
    if (a->pool == GL_POOL_MAX) {
      GL_TRY(launch_fwd_any<PK_MAX>(a->act, a->K, a->D, k, s));
      GL_LAUNCH(GL_KERNEL_FWD_FINALIZE, fwd_finalize_max_kernel, grid, dim3(256), 0, s, part, pslot, pre, winner, Bc,
                a->G, q.cpg, b_pad);
    } else if (a->pool == GL_POOL_TOPK_MEAN) {
      GL_TRY(launch_fwd_any<PK_TOPK>(a->act, a->K, a->D, k, s));
      const dim3 g1((unsigned)ceil_div((long long)Bc * a->G, 256));
      const bool top8 = a->topk == 8 && q.cpg <= FWD_TOP8_CPG && ((uintptr_t)winner & 15) == 0;
      if (top8 && a->act == GL_ACT_RELU)
        GL_LAUNCH(GL_KERNEL_FWD_FINALIZE, fwd_finalize_top8_kernel<GL_ACT_RELU>, g1, dim3(256), 0, s, part, pslot,
                  a->counts, pre, winner, Bc, a->G, q.cpg, b_pad);
      else if (top8 && a->act == GL_ACT_GELU)
        GL_LAUNCH(GL_KERNEL_FWD_FINALIZE, fwd_finalize_top8_kernel<GL_ACT_GELU>, g1, dim3(256), 0, s, part, pslot,
                  a->counts, pre, winner, Bc, a->G, q.cpg, b_pad);
      else if (top8)
        GL_LAUNCH(GL_KERNEL_FWD_FINALIZE, fwd_finalize_top8_kernel<GL_ACT_IDENTITY>, g1, dim3(256), 0, s, part, pslot,
                  a->counts, pre, winner, Bc, a->G, q.cpg, b_pad);
      else if (a->act == GL_ACT_RELU)
        GL_LAUNCH(GL_KERNEL_FWD_FINALIZE, fwd_finalize_topk_kernel<GL_ACT_RELU>, g1, dim3(256), 0, s, part, pslot,
                  a->counts, pre, winner, Bc, a->G, q.cpg, b_pad, a->topk);
      else if (a->act == GL_ACT_GELU)
        GL_LAUNCH(GL_KERNEL_FWD_FINALIZE, fwd_finalize_topk_kernel<GL_ACT_GELU>, g1, dim3(256), 0, s, part, pslot,
                  a->counts, pre, winner, Bc, a->G, q.cpg, b_pad, a->topk);
      else
        GL_LAUNCH(GL_KERNEL_FWD_FINALIZE, fwd_finalize_topk_kernel<GL_ACT_IDENTITY>, g1, dim3(256), 0, s, part, pslot,
                  a->counts, pre, winner, Bc, a->G, q.cpg, b_pad, a->topk);
    } else if (pool_smooth(a->pool)) {
      const dim3 g1((unsigned)ceil_div((long long)Bc * a->G, 256));
      float* lse = a->lse ? a->lse + (long long)b0 * a->G : nullptr;
      if (a->pool == GL_POOL_LME) {
        GL_TRY(launch_fwd_any<PK_LME>(a->act, a->K, a->D, k, s));
        GL_LAUNCH(GL_KERNEL_FWD_FINALIZE, fwd_finalize_smooth_kernel<SM_LME>, g1, dim3(256), 0, s, part, a->counts, pre,
                  lse, Bc, a->G, q.cpg, b_pad, k.scale, k.pparam, k.pint);
      } else if (a->pool == GL_POOL_POWER) {
        switch (k.pint) {  // a kernel per integer p (12 waves per workgroup at K = 8)
          case 1: GL_TRY(launch_fwd_any<PK_POW_I + 1>(a->act, a->K, a->D, k, s)); break;
          case 2: GL_TRY(launch_fwd_any<PK_POW_I + 2>(a->act, a->K, a->D, k, s)); break;
          case 4: GL_TRY(launch_fwd_any<PK_POW_I + 4>(a->act, a->K, a->D, k, s)); break;
          case 8: GL_TRY(launch_fwd_any<PK_POW_I + 8>(a->act, a->K, a->D, k, s)); break;
          default: GL_TRY(launch_fwd_any<PK_POW>(a->act, a->K, a->D, k, s));
        }
        GL_LAUNCH(GL_KERNEL_FWD_FINALIZE, fwd_finalize_smooth_kernel<SM_POW>, g1, dim3(256), 0, s, part, a->counts, pre,
                  lse, Bc, a->G, q.cpg, b_pad, k.scale, k.pparam, k.pint);
      } else {
        GL_TRY(launch_fwd_any<PK_SW>(a->act, a->K, a->D, k, s));
        GL_LAUNCH(GL_KERNEL_FWD_FINALIZE, fwd_finalize_smooth_kernel<SM_SW>, g1, dim3(256), 0, s, part, a->counts, pre,
                  lse, Bc, a->G, q.cpg, b_pad, k.scale, k.pparam, k.pint);
      }
    } else {
      GL_TRY(launch_fwd_any<PK_SUM>(a->act, a->K, a->D, k, s));
      GL_LAUNCH(GL_KERNEL_FWD_FINALIZE, fwd_finalize_kernel, grid, dim3(256), 0, s, part, a->counts, pre, Bc, a->G,
                q.cpg, b_pad, 0, a->pool);
    }
    GL_CHECK_LAUNCH();
  }
  return 0;
}

// ---- the forward without a caller workspace ----------------------------------------------------
// gl_fwd_static keeps its token tiles and partial results in this file-scope device array (one
// copy per GPU, held until the process ends) instead of a caller workspace, for callers that cannot
// allocate.  Host code never passes the array's name to a kernel: it passes the per-device address
// that hipGetSymbolAddress returns.  The forward runs as many token passes as the array needs; the
// results are those of gl_fwd (every token's arithmetic and order are the same).
static __device__ __align__(256) unsigned char scratch[GL_FWD_STATIC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];       // per device; null until resolved
hipEvent_t g_scratch_last[kMaxScratchDevices];  // per device: recorded after the last use's launches
bool g_scratch_used[kMaxScratchDevices];
}  // namespace

// the address of this device's scratch and its "last use" event (resolved once per device, with
// the device current); call with g_scratch_mu held
static int scratch_address(int* dev_out, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) return GL_ERR_DEVICE;
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return GL_ERR_DEVICE;
    e = hipEventCreateWithFlags(&g_scratch_last[dev], hipEventDisableTiming);
    if (e != hipSuccess) return (int)e;
    g_scratch_ptr[dev] = p;
  }
  *dev_out = dev;
  *out = g_scratch_ptr[dev];
  return 0;
}

// the largest token chunk whose tiles and partials fit the scratch (0: not even one tile)
static long long static_chunk(const GlFwdArgs* a) {
  const long long cpg = ceil_div(a->S, 64 * FWD_NPL);
  const long long per_token = fwd_part_per_token(a, (long long)a->G * cpg) + (long long)a->D * 4;
  const long long room = (long long)GL_FWD_STATIC_SCRATCH_BYTES - 3 * 256;  // three sections rounded to 256
  return room / per_token / BT * BT;
}

}  // namespace gl

using namespace gl;

extern "C" int gl_fwd_workspace(const GlFwdArgs* a, size_t* bytes) {
  if (!a || !bytes) return GL_ERR_ARG;
  GL_TRY(check_layer(a->B, a->D, a->G, a->S, a->K, a->act, a->pool, a->X, a->idx, a->W, a->bias, a->counts,
                     a->x_dtype, a->w_dtype));
  GL_TRY(check_topk(a->pool, a->topk, a->S));
  GL_TRY(check_rec_shift(a->rec_shift, a->S, a->sched));
  GL_TRY(check_smooth(a->pool, a->pool_param, a->act));
  int32_t sps = a->sps, gs = a->gs;
  GL_TRY(check_geometry(a->G, a->S, &sps, &gs));
  if (sps > 1 && a->rec_shift > 0) return GL_ERR_UNSUPPORTED;
  FwdPlan q = fwd_plan(a);
  *bytes = q.xt_bytes + q.part_bytes + q.slot_bytes;
  return 0;
}

extern "C" int gl_fwd_mask_bytes(const GlFwdArgs* a, size_t* bytes) {
  if (!a || !bytes) return GL_ERR_ARG;
  *bytes = relu_mask_layer(a->act, a->pool, a->K, a->rec_shift, a->x_dtype, a->D) && a->B > 0 && a->G > 0 && a->S > 0
               ? relu_mask_bytes(a->G, a->S, a->B)
               : 0;
  return 0;
}

extern "C" int gl_fwd(const GlFwdArgs* a, void* stream) {
  if (!a || !a->pre) return GL_ERR_ARG;
  if (a->relu_mask && !relu_mask_layer(a->act, a->pool, a->K, a->rec_shift, a->x_dtype, a->D)) return GL_ERR_ARG;
  size_t need = 0;
  GL_TRY(gl_fwd_workspace(a, &need));
  if (!a->ws || a->ws_bytes < need) return GL_ERR_WORKSPACE;
  if (a->sched && a->K != 8) return GL_ERR_UNSUPPORTED;
  return fwd_run(a, a->ws, fwd_plan(a), (hipStream_t)stream);
}

extern "C" int gl_fwd_static(const GlFwdArgs* a, void* stream) {
  if (!a || !a->pre) return GL_ERR_ARG;
  if (a->relu_mask && !relu_mask_layer(a->act, a->pool, a->K, a->rec_shift, a->x_dtype, a->D)) return GL_ERR_ARG;
  size_t need = 0;
  GL_TRY(gl_fwd_workspace(a, &need));  // argument checks; ws / ws_bytes are ignored
  if (a->sched && a->K != 8) return GL_ERR_UNSUPPORTED;
  const long long bf = static_chunk(a);
  if (bf < BT) return GL_ERR_SCRATCH;
  const FwdPlan q = fwd_plan(a, bf);
  if (q.xt_bytes + q.part_bytes + q.slot_bytes > (size_t)GL_FWD_STATIC_SCRATCH_BYTES) return GL_ERR_SCRATCH;
  // Calls on one GPU share its scratch.  A call waits on the device's "last use" event before its
  // launches and records it after them, so calls on different streams of one GPU run one after
  // the other instead of overwriting each other's tiles.  Under graph capture the event is left
  // alone: the captured graph's own dependencies order its nodes.
  const hipStream_t s = (hipStream_t)stream;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  int dev = -1;
  void* ws = nullptr;
  GL_TRY(scratch_address(&dev, &ws));
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &cap);
  if (e != hipSuccess) return (int)e;
  const bool order = cap == hipStreamCaptureStatusNone;
  if (order && g_scratch_used[dev]) {
    e = hipStreamWaitEvent(s, g_scratch_last[dev], 0);
    if (e != hipSuccess) return (int)e;
  }
  GL_TRY(fwd_run(a, ws, q, s));
  if (order) {
    e = hipEventRecord(g_scratch_last[dev], s);
    if (e != hipSuccess) return (int)e;
    g_scratch_used[dev] = true;
  }
  return 0;
}
