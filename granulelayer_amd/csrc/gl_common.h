// Shared definitions of the granulelayer_amd HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "../../include/granulelayer_amd.h"

namespace gl {

// ---- tiling constants ---------------------------------------------------------------------
// X is staged feature-major in LDS, 4 tokens per 16-byte slot: one ds_read_b128 gathers one
// input feature for 4 tokens.
constexpr int BT = 4;
// dX: features per range (one accumulator row each) and slots per edge-list unit.
constexpr int FW = 8;
constexpr int US = 1024;
// dX edge record (32 bit): bits [0, 16) byte offset of W[n, k] inside its unit,
// (s_local * K + k) * 4; bits [16, 24) feature inside the range; bit 31 set when the feature
// differs from the one of the previous edge of the same segment (a new accumulation run).
constexpr int REC_F_SHIFT = 16;
constexpr unsigned REC_OFF_MASK = 0xffffu;
constexpr unsigned REC_F_MASK = 0xffu;
constexpr unsigned REC_NEWF = 1u << 31;
// largest token chunk of one backward pass (bounds the per-neuron mask record)
constexpr int BWD_TOKEN_CHUNK = 1024;

constexpr int ceil_div(long long a, long long b) { return (int)((a + b - 1) / b); }

// ---- gather schedule of the neuron-stationary kernels (gl_sched.hip) --------------------------
// Slots are scheduled in windows of 128: neuron slot j of lane `lane` in a chunk starting at slot
// s_lo (a multiple of 64) lies in half-window h = s_lo / 64 + j and reads record
// ((g * nwin + h / 2) * 128 + ((h % 2) * 4 + lane / 16) * 16 + lane % 16) = s_local | k_0 << 7 |
// ... | k_6 << 25 (k_7 = 28 - sum).  Without a schedule the slot is s_lo + 64 j + lane and edges
// are visited in k order.
constexpr int SCHED_WIN = 128;
constexpr uint32_t SCHED_IDENTITY = 0u | 1u << 3 | 2u << 6 | 3u << 9 | 4u << 12 | 5u << 15 | 6u << 18;

// slot (within the pool; >= S when the window lies past the pool) and packed visiting order
__device__ __forceinline__ int sched_slot(const uint32_t* __restrict__ sched, int nwin, int S, long long g, int s_lo,
                                          int j, int lane, uint32_t& order) {
  if (sched == nullptr) {
    order = SCHED_IDENTITY;
    return s_lo + j * 64 + lane;
  }
  // neuron j of the chunk is half-window h = s_lo / 64 + j (chunks start at multiples of 64 slots);
  // half h % 2 of window h / 2 holds its 64 lanes' records
  const int h = (s_lo >> 6) + j;
  const int w = h >> 1;
  if (w >= nwin) {
    order = SCHED_IDENTITY;
    return S;
  }
  const uint32_t rec = sched[((long long)g * nwin + w) * SCHED_WIN + ((h & 1) * 4 + (lane >> 4)) * 16 + (lane & 15)];
  order = rec >> 7;
  return w * SCHED_WIN + (int)(rec & 127u);
}

// edge visited at position ks (K = 8 orders; K = 16 is never scheduled)
template <int K>
__device__ __forceinline__ int sched_k(uint32_t order, int ks) {
  if constexpr (K != 8) {
    return ks;
  } else {
    if (ks < 7) return (int)((order >> (3 * ks)) & 7u);
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 7; ++i) sum += (int)((order >> (3 * i)) & 7u);
    return 28 - sum;
  }
}
constexpr long long round_up(long long a, long long b) { return (a + b - 1) / b * b; }

// ---- where a pool's slots live --------------------------------------------------------------
// Pools are the groups (sps <= 1: pool g's S slots start at neuron g * S), or, for two-level
// pooling, the sps level-1 shards of each group: pool u is shard u % sps of group u / sps, its
// slots start at (u % sps) * S inside a group of gs slots, and the group's last shard may end
// inside the group (gs < sps * S), which pool_ext reports.  Pool-indexed data (counts, partials,
// schedules, windows) is per pool; neuron-indexed data (idx, W, bias, dW, db, masks) is per
// physical neuron.
__host__ __device__ __forceinline__ long long pool_base(int g, int S, int sps, int gs) {
  return sps <= 1 ? (long long)g * S : (long long)(g / sps) * gs + (long long)(g % sps) * S;
}
// slots of pool g inside its group (>= 1): the clamp target of padded slots' addresses
__host__ __device__ __forceinline__ int pool_ext(int g, int S, int sps, int gs) {
  if (sps <= 1) return S;
  const int r = gs - (g % sps) * S;
  return r < S ? r : S;
}

// input k of neuron n when 2^rs consecutive slots share one index record (rs = 0: own record)
__device__ __forceinline__ int rec_index(const int32_t* __restrict__ idx, long long n, int k, int K, int rs) {
  return idx[(n >> rs) * K + k];
}

// ---- parameters stored as fp32 or bf16 ------------------------------------------------------------
// W and bias are read in their stored dtype and widened in the kernel (bf16 -> fp32 is exact: the
// 16 bits become the high half of the fp32 pattern), as the reference's kernels load W[nk] and
// widen it (triton_fused.py:257).  With bf, p points at bf16 elements.
__device__ __forceinline__ float ld_param(const float* p, bool bf, long long i) {
  if (bf) return __uint_as_float((unsigned)reinterpret_cast<const unsigned short*>(p)[i] << 16);
  return p[i];
}
// The same with the dtype fixed at compile time: loops of parameter loads are instantiated once per
// dtype behind one uniform branch (a dtype test per load keeps the compiler from batching them)
template <bool BF>
__device__ __forceinline__ float ld_param_t(const float* p, long long i) {
  if constexpr (BF) return __uint_as_float((unsigned)reinterpret_cast<const unsigned short*>(p)[i] << 16);
  return p[i];
}
// the fp32 value of a weight whose 32-bit word w32 was loaded from byte offset (boff & ~3) of bf16
// storage (boff = the element's byte offset): its half of the word
__device__ __forceinline__ float bf16_half(unsigned w32, unsigned boff) {
  return __uint_as_float((boff & 2u) ? (w32 & 0xffff0000u) : (w32 << 16));
}

// ---- the neuron activation and its derivative (triton_fused.py:29-45 _act / _dact) -------------
// GELU is the exact (erf) form, 0.5 z (1 + erf(z / sqrt 2)), with derivative Phi(z) + z phi(z).
// -inf (the max tile's padded-slot sentinel) stays -inf under every activation.
template <int ACT>
__device__ __forceinline__ float act_f(float z) {
  if constexpr (ACT == GL_ACT_RELU) {
    return __builtin_fmaxf(z, 0.f);
  } else if constexpr (ACT == GL_ACT_GELU) {
    const float g = 0.5f * z * (1.f + erff(z * 0.70710678118654752f));
    return z == -__builtin_inff() ? z : g;
  } else {
    return z;
  }
}
template <int ACT>
__device__ __forceinline__ float dact_f(float z) {
  if constexpr (ACT == GL_ACT_RELU) {
    return z > 0.f ? 1.f : 0.f;
  } else if constexpr (ACT == GL_ACT_GELU) {
    const float cdf = 0.5f * (1.f + erff(z * 0.70710678118654752f));
    return __builtin_fmaf(z * 0.39894228040143268f, expf(-0.5f * z * z), cdf);
  } else {
    return 1.f;
  }
}

// Tokens of one dX wave: 64 lanes x T slots, T in {1, 2, 4}, for a chunk of B tokens.
inline int dx_slots(int B) { return B <= 64 ? 1 : (B <= 128 ? 2 : 4); }
inline int dx_cap(int B) { return (int)round_up(B, 64 * dx_slots(B)); }
// per-neuron activation-mask record of the backward: one bit per token of the padded chunk
// (an even number of 32-bit words: the dX kernel reads 64-bit words)
inline int mask_stride(int B) { return dx_cap(B) / 32; }

#define GL_CHECK_LAUNCH()                                   \
  do {                                                      \
    hipError_t e_ = hipGetLastError();                      \
    if (e_ != hipSuccess) return (int)e_;                   \
  } while (0)

#define GL_TRY(x)                                           \
  do {                                                      \
    int r_ = (x);                                           \
    if (r_ != 0) return r_;                                 \
  } while (0)

__device__ __forceinline__ float load_x(const float* p, long long i) { return p[i]; }
__device__ __forceinline__ float load_x(const __hip_bfloat16* p, long long i) {
  // bf16 -> fp32 is exact: the 16 bits become the high half of the fp32 pattern
  unsigned short u = reinterpret_cast<const unsigned short*>(p)[i];
  return __uint_as_float((unsigned)u << 16);
}

// A copy of v the optimiser cannot see through: address arithmetic that depends on it is
// computed where it is used instead of being hoisted out of the token loop and kept live in
// registers for the whole kernel.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// ---- X token tiles: global -> LDS directly ----------------------------------------------------
// A tile is D float4 slots (4 tokens per input feature).  Every lane copies 16-byte slots with
// global_load_lds_dwordx4, which writes lane i's data to LDS at (wave-uniform base) + 16 i, so the
// data never passes through VGPRs.  D <= XTILE_DB features: two static buffers, the next tile
// lands while the current one is read; larger D (up to XTILE_SB): one buffer; wider layers
// gather from the token tiles in global memory (the XG kernel variants).
constexpr int XTILE_DB = 4096;
constexpr int XTILE_SB = 10112;

// The copy is issued from inline asm: the compiler does not see these loads, so it inserts no
// vmcnt wait for them before LDS reads of the tile buffers, and its LDS-read waits stay graded
// (lgkmcnt(n) for the reads a use needs; the builtin global_load_lds makes it wait for every
// outstanding LDS read, and for the copy itself before any read of the same LDS object).  The
// caller waits with stage_wait() and a barrier before reading the tile.
// A wave-uniform global address in scalar registers.  readfirstlane is 32-bit and returns int:
// the halves go through it separately and are widened as unsigned (a sign-extended low half would
// set every bit of the high half whenever bit 31 of the address is set).
__device__ __forceinline__ const char* uniform_ptr(const void* p) {
  const unsigned long long a = (unsigned long long)(size_t)p;
  const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((unsigned)a);
  const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
  return (const char*)(size_t)((unsigned long long)hi << 32 | (unsigned long long)lo);
}
__device__ __forceinline__ void dma_tile(const float4* __restrict__ src, float4* dst, int D, int nthreads) {
  // Pass r copies slots [r * nthreads, (r + 1) * nthreads): the pass base is wave-uniform and
  // goes into the scalar address and M0; the lane part is the one VGPR threadIdx.x * 16.
  const unsigned tid = threadIdx.x;
  const unsigned wave0 = __builtin_amdgcn_readfirstlane(tid & ~63u);  // thread index of the wave's lane 0
  const char* s0 = uniform_ptr(src);
  const unsigned d0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)dst);
  for (int b = 0; b < D; b += nthreads) {
    if (b + (int)tid < D) {
      const char* sb = s0 + (size_t)b * 16;
      const unsigned m0v = d0 + (unsigned)(b + (int)wave0) * 16u;
      asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %2"
                   :: "v"(tid * 16u), "s"(m0v), "s"(sb) : "memory", "m0");
    }
  }
}
// ---- pool-window staging -----------------------------------------------------------------------
// When the pools of every workgroup draw their inputs from narrow windows (gl_window_build_host),
// the forward and dW kernels stage only those windows: a stage is WS_TILES token tiles, each
// [pool k of the workgroup][window slot i] with nsl = npw * ww slots of 16 bytes (npw pools per
// workgroup, ww the widest window rounded up to 64), slot (k, i) = X[tile][lo_k + i].  Two stage
// regions of WS_TILES * nsl slots alternate; tile t sits at slot (t mod 2 WS_TILES) * nsl, so the
// kernels step their LDS addresses by nsl * 16 bytes per tile.  nsl <= WS_SLOTS keeps a region in
// 64 KiB; one barrier serves WS_TILES tiles.
constexpr int WS_TILES = 4;
constexpr int WS_SLOTS = XTILE_DB / WS_TILES;

struct WinLayout {
  const uint32_t* win;  // [G] first input of each pool's window
  int ww, npw, g_first, G;
};

// region <- the WS_TILES tiles from t0 (tiles past n_tiles repeat the last one: in bounds, unread).
// A stage is WS_TILES * npw runs (one tile's window of one pool, ww slots); wave w copies runs
// w, w + waves, ...  (taking its own runs directly: walking every 64-slot group of the stage in
// each wave cost ~25% of the kernel in scalar instructions)
// IB: bytes per input of the tiles (16: 4 fp32 tokens; 8: 4 raw bf16 tokens, where the window
// starts at the even input at or below lo so every copied 16-byte slot is a whole slot of the tile).
template <int IB = 16>
__device__ __forceinline__ void dma_window_stage(const float4* __restrict__ xt, float4* region, int t0, int n_tiles,
                                                 int D, const WinLayout& L, int waves) {
  constexpr int IPS = 16 / IB;  // inputs per 16-byte slot
  const unsigned lane = threadIdx.x & 63u;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const char* xb = uniform_ptr(xt);
  const unsigned r0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)region);
  const int nsl = L.ww / IPS, last = D / IPS - 1;  // slots per run; the tile's last slot (D even when IPS = 2)
  for (int run = wave; run < WS_TILES * L.npw; run += waves) {
    const int tt = run / L.npw, k = run - tt * L.npw;
    const int t = t0 + tt < n_tiles ? t0 + tt : n_tiles - 1;
    const int g = L.g_first + k < L.G ? L.g_first + k : L.G - 1;
    const int lo = (int)__builtin_amdgcn_readfirstlane(L.win[g]) / IPS;  // first slot of the window
    const char* sb = xb + (size_t)t * D * IB;
    for (int i0 = 0; i0 < nsl; i0 += 64) {
      // nsl is a multiple of 64 for 16-byte inputs, of 32 for 8-byte ones: lanes past the run
      // write nothing
      if (i0 + (int)lane >= nsl) continue;
      const int col = lo + i0 + (int)lane < last ? lo + i0 + (int)lane : last;
      const unsigned m0v = r0 + (unsigned)(run * nsl + i0) * 16u;
      asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %2"
                   :: "v"((unsigned)col * 16u), "s"(m0v), "s"(sb) : "memory", "m0");
    }
  }
}
// LDS byte address of input d of a neuron in pool slot k of the workgroup whose window starts at lo
// (IB bytes per input; with IB = 8 the staged window starts at the even input lo & ~1)
template <int IB = 16>
__device__ __forceinline__ unsigned win_addr(int d, int k, int lo, int ww) {
  if constexpr (IB == 8) lo &= ~1;
  int i = d - lo;
  i = i < 0 ? 0 : (i >= ww ? ww - 1 : i);  // the host validated the widths; clamp keeps LDS reads in bounds
  return (unsigned)(k * ww + i) * (unsigned)IB;
}

// Four consecutive floats at a wave-uniform address, read through the constant address space so
// the load stays scalar (s_load) even after barriers and LDS-DMA, where a generic load of the
// same address becomes a vector load the vmcnt waits then include.
__device__ __forceinline__ float4 ld_uniform4(const float* row, int i) {
  typedef const __attribute__((address_space(4))) float CF;
  const CF* q = (const CF*)(row + i);
  return make_float4(q[0], q[1], q[2], q[3]);
}
// X slot at byte offset a of a tile buffer.  FAR: the buffer's base does not fit the 16-bit
// ds_read offset, so base + a costs one v_add per read; the offset then passes through an empty
// asm so the compiler keeps doing that add at the read instead of hoisting a second copy of every
// address out of the tile loop (which would not fit the register file).
template <bool FAR>
__device__ __forceinline__ float4 gather_x(const char* buf, unsigned a) {
  if constexpr (FAR) asm volatile("" : "+v"(a));
  return *reinterpret_cast<const float4*>(buf + a);
}
// The same gather from a token tile in global memory (the XG kernels, D > XTILE_SB): a buffer
// resource over the tile (wave-uniform, in SGPRs) and the slot's 32-bit byte offset, one
// buffer_load_dwordx4 per read with no 64-bit address arithmetic; reads past the tile return 0.
struct XBuf {
  __amdgpu_buffer_rsrc_t r;
};
__device__ __forceinline__ XBuf xbuf(const float4* tile, int D) {
  // dword 3 0x00020000: raw 32-bit data, the gfx9 buffer format of untyped loads
  return XBuf{__builtin_amdgcn_make_buffer_rsrc(const_cast<float4*>(tile), (short)0, D * 16, 0x00020000)};
}
// A load from a wave-uniform base address plus the lane's 32-bit byte offset, as one buffer load:
// the base goes into scalar registers (readfirstlane, then a buffer resource without a range
// limit) and the lane supplies only the offset, so no 64-bit vector address arithmetic is needed.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(uniform_ptr(base)), (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ unsigned ld_uniform_u32(const void* base, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b32(uniform_rsrc(base), (int)off, 0, 0);
}
__device__ __forceinline__ uint2 ld_uniform_u64(const void* base, unsigned off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(uniform_rsrc(base), (int)off, 0, 0);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint4 ld_uniform_u128(const void* base, unsigned off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(uniform_rsrc(base), (int)off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Two-token tiles (8-byte slots, D x 8 bytes per tile): tokens 2t, 2t + 1 of input d at byte 8 d.
// Inputs up to 2 XTILE_DB fit one 64-KiB buffer, so the wider layers keep two buffers (or two
// workgroups) per CU; the price is twice the tiles, reductions and barriers per token.
template <bool FAR>
__device__ __forceinline__ float2 gather_x2(const char* buf, unsigned a) {
  if constexpr (FAR) asm volatile("" : "+v"(a));
  return *reinterpret_cast<const float2*>(buf + a);
}
__device__ __forceinline__ float2 ld_uniform2(const float* row, int i) {
  typedef const __attribute__((address_space(4))) float CF;
  const CF* q = (const CF*)(row + i);
  return make_float2(q[0], q[1]);
}

template <bool FAR>
__device__ __forceinline__ float4 gather_x(XBuf b, unsigned a) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(b.r, (int)a, 0, 0);
  return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
}
// this wave's tile loads have reached LDS (vmcnt(0)); a barrier then publishes every wave's
__device__ __forceinline__ void stage_wait() { __builtin_amdgcn_s_waitcnt(0x3f70); }

// DPP move (row/quad patterns) as a float; the source lane is always valid for the patterns used
// here, so the move folds into the consuming v_add_f32 as a DPP operand
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Token of a tile whose total wave_sum4 leaves in lane l (l mod 4 = 0, 1, 2, 3 -> 0, 2, 1, 3).
__device__ __forceinline__ int wave_sum4_token(int lane) { return ((lane & 1) << 1) | ((lane >> 1) & 1); }

// Sums over the 64 lanes of a wave of four per-lane values (one per token of a tile), as a
// reduce-scatter: two quad steps leave each lane one token's quad sum (lane ^ 1: even lanes keep
// tokens 0, 1, odd lanes 2, 3; lane ^ 2: one of the two), two row rotations sum the 4 quads of a
// row with the same token, and the two cross-row swaps of gfx950 (v_permlane16_swap rows 0<->1,
// 2<->3, v_permlane32_swap rows 0,1<->2,3) add the rows.  Every lane ends with the total of token
// wave_sum4_token(lane).  VALU only (no LDS round trips), fixed order: deterministic.
__device__ __forceinline__ float wave_sum4(float a0, float a1, float a2, float a3, int lane) {
  const bool odd = lane & 1, hi = lane & 2;
  const float b0 = (odd ? a2 : a0) + dpp<0xB1>(odd ? a0 : a2);  // quad_perm(1,0,3,2)
  const float b1 = (odd ? a3 : a1) + dpp<0xB1>(odd ? a1 : a3);
  float c = (hi ? b1 : b0) + dpp<0x4E>(hi ? b0 : b1);  // quad_perm(2,3,0,1)
  c += dpp<0x124>(c);  // row_ror:4
  c += dpp<0x128>(c);  // row_ror:8
  // each swap returns (first operand with its odd rows / rows 2,3 replaced, second operand with
  // its even rows / rows 0,1 replaced); with both operands c their sum holds the row-pair sum
  const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(c), __float_as_uint(c), false, false);
  c = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
  const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(c), false, false);
  return __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
}

// The same reduction for two per-lane values (two-token tiles): after the first quad step even
// lanes hold token 0 and odd lanes token 1; the remaining steps pair lanes of equal parity.
// Every lane ends with the total of token lane & 1.
__device__ __forceinline__ float wave_sum2(float a0, float a1, int lane) {
  const bool odd = lane & 1;
  float c = (odd ? a1 : a0) + dpp<0xB1>(odd ? a0 : a1);  // quad_perm(1,0,3,2)
  c += dpp<0x4E>(c);   // quad_perm(2,3,0,1)
  c += dpp<0x124>(c);  // row_ror:4
  c += dpp<0x128>(c);  // row_ror:8
  const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(c), __float_as_uint(c), false, false);
  c = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
  const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(c), false, false);
  return __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
}

// Max pooling keeps (value, slot) pairs ordered by value, then by the smaller slot: the maximum
// of act(z) and the first slot reaching it (torch.argmax).  The order is total (for non-NaN
// values), so any combination order gives the same pair.
__device__ __forceinline__ void vmax_pair(float& m, int& s, float m2, int s2) {
  const bool take = m2 > m || (m2 == m && s2 < s);
  m = take ? m2 : m;
  s = take ? s2 : s;
}

template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

// wave_sum4's reduce-scatter for (value, slot) pairs: every lane ends with the wave's maximum
// pair of token wave_sum4_token(lane).
__device__ __forceinline__ void wave_max4(float a0, float a1, float a2, float a3, int s0, int s1, int s2, int s3,
                                          int lane, float& m, int& s) {
  const bool odd = lane & 1, hi = lane & 2;
  float b0 = odd ? a2 : a0, b1 = odd ? a3 : a1;
  int t0 = odd ? s2 : s0, t1 = odd ? s3 : s1;
  vmax_pair(b0, t0, dpp<0xB1>(odd ? a0 : a2), dppi<0xB1>(odd ? s0 : s2));  // quad_perm(1,0,3,2)
  vmax_pair(b1, t1, dpp<0xB1>(odd ? a1 : a3), dppi<0xB1>(odd ? s1 : s3));
  float c = hi ? b1 : b0;
  int u = hi ? t1 : t0;
  vmax_pair(c, u, dpp<0x4E>(hi ? b0 : b1), dppi<0x4E>(hi ? t0 : t1));  // quad_perm(2,3,0,1)
  vmax_pair(c, u, dpp<0x124>(c), dppi<0x124>(u));                      // row_ror:4
  vmax_pair(c, u, dpp<0x128>(c), dppi<0x128>(u));                      // row_ror:8
  const auto c16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(c), __float_as_uint(c), false, false);
  const auto u16 = __builtin_amdgcn_permlane16_swap((unsigned)u, (unsigned)u, false, false);
  c = __uint_as_float(c16[0]);
  u = (int)u16[0];
  vmax_pair(c, u, __uint_as_float(c16[1]), (int)u16[1]);
  const auto c32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(c), false, false);
  const auto u32 = __builtin_amdgcn_permlane32_swap((unsigned)u, (unsigned)u, false, false);
  m = __uint_as_float(c32[0]);
  s = (int)u32[0];
  vmax_pair(m, s, __uint_as_float(c32[1]), (int)u32[1]);
}

// ---- smooth pooling states (LogMeanExp, power mean, softmax-weighted) ---------------------------
// LogMeanExp / softmax-weighted keep (m, s, t) per token: m the largest u = a * scale, s = sum 2^(u - m),
// t = sum 2^(u - m) a (softmax-weighted only); power mean keeps m the largest a and s = sum (a / m)^p.
// Two states merge by rescaling to the larger m (kernels/triton_fused.py:180-222 restated as a
// pairwise merge); an empty state has m = -inf (exp2 forms) or m = 0 (power).
constexpr int SM_LME = 0, SM_POW = 1, SM_SW = 2;
// the dense-dz backward of sum / mean pooling with a GELU neuron activation (dz = c1 gelu'(z), no
// 0 / 1 mask): SM_LIN is its operator in the smooth pools' recompute kernel
constexpr int SM_LIN = 3;

// q^p for q >= 0: exact products for p in {1, 2, 4, 8} (pint), else exp2(p log2 q)
__device__ __forceinline__ float pow_p(float q, float p, int pint) {
  if (pint == 1) return q;
  if (pint == 2) return q * q;
  if (pint == 4) { const float q2 = q * q; return q2 * q2; }
  if (pint == 8) { const float q2 = q * q, q4 = q2 * q2; return q4 * q4; }
  return q > 0.f ? __builtin_amdgcn_exp2f(p * __builtin_amdgcn_logf(q)) : 0.f;
}

template <int OP>
__device__ __forceinline__ void sm_merge(float& m, float& s, float& t, float m2, float s2, float t2, float p, int pint) {
  if constexpr (OP == SM_POW) {
    const float M = __builtin_fmaxf(m, m2);
    const float inv = M > 0.f ? 1.f / M : 0.f;
    s = M > 0.f ? s * pow_p(m * inv, p, pint) + s2 * pow_p(m2 * inv, p, pint) : 0.f;
    m = M;
  } else {
    const float M = __builtin_fmaxf(m, m2);
    const float base = M == -__builtin_inff() ? 0.f : M;  // both empty: keep s = t = 0
    const float r1 = __builtin_amdgcn_exp2f(m - base), r2 = __builtin_amdgcn_exp2f(m2 - base);
    s = s * r1 + s2 * r2;
    if constexpr (OP == SM_SW) t = t * r1 + t2 * r2;
    m = M;
  }
}

}  // namespace gl
