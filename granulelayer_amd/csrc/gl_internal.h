// Internal declarations shared by the library's translation units.
#pragma once

#include "gl_common.h"

namespace gl {

// LDS available to one workgroup on the current device (queried once per device).
size_t max_lds_bytes();
// Raise a kernel's dynamic-LDS limit when it needs more than the 64 KiB default.
int set_lds_limit(const void* kernel, size_t bytes);

int check_layer(int B, int D, int G, int S, int K, int act, int pool, const void* X, const int32_t* idx, const void* W,
                const void* bias, const int32_t* counts, int x_dtype, int w_dtype);

// GL_POOL_TOPK_MEAN arguments (k, pool size); 0 for other pools
int check_topk(int pool, int topk, int S);

// smooth pools' parameter (temperature, p with relu activations, beta)
int check_smooth(int pool, float param, int act);

// shared index records: 0 <= rec_shift <= 4, S a multiple of 2^rec_shift, no gather schedule
int check_rec_shift(int rec_shift, int S, const void* sched);

// Pool geometry (pool_base): *sps <= 1 becomes 1 with *gs = S (pools are groups; a given *gs must
// equal S); otherwise G a multiple of *sps and (*sps - 1) * S < *gs <= *sps * S, so every shard
// starts inside its group.
int check_geometry(int G, int S, int32_t* sps, int32_t* gs);

// Window staging for a kernel whose workgroups hold `waves` chunks of cpg per pool: true (with the
// padded width *ww and pools per workgroup *npw) when the pools' windows fit a stage tile.
// max_slots: the 16-byte slots one token tile of the stage may take (WS_SLOTS: two regions fill 128 KiB);
// in_bytes: bytes per staged input (16: 4 fp32 tokens; 8: 4 bf16 tokens, windows from an even input).
bool window_staging(const uint32_t* win, int width, int D, int waves, int cpg, int G, int* ww, int* npw,
                    int max_slots = WS_SLOTS, int in_bytes = 16);

// X rows [b0, b0 + n_tiles*tb) -> token tiles [n_tiles][D] of tb floats (zero past B): float4
// slots (tb = 4) or the two-token float2 slots (tb = 2).  The same bytes either way.
int launch_tile_x(const void* X, long long sxb, int x_dtype, int B, int D, int b0, int n_tiles, float4* xt,
                  hipStream_t s, int tb = 4);

// bf16 X rows [b0, b0 + 4 n_tiles) -> 4-token tiles [n_tiles][D] of raw bf16 bits in 8 bytes
// (word 0 = token 1 << 16 | token 0, word 1 = token 3 << 16 | token 2; +0 past B).
int launch_tile_x_bf16x4(const void* X, long long sxb, int B, int D, int b0, int n_tiles, void* xt, hipStream_t s);

// Two-token tiles (tb = 2) for the inputs past one 16-byte-slot buffer: XTILE_DB < D <= 2 XTILE_DB, D even.
inline bool tiles_of_two(int D) { return D > XTILE_DB && D <= 2 * XTILE_DB && D % 2 == 0; }

// The forward's ReLU bits for the backward (GlFwdArgs / GlBwdArgs.relu_mask): ReLU mean / sum at
// K = 8, where the forward and the dW pass both give a wave a chunk of RELU_MASK_NPL x 64 slots of
// one pool with the same lane / slot assignment (sched_slot), one record per slot, and 4-token X
// tiles in both passes (fp32 X over 4097..8192 inputs runs two-token tiles).  Layout: per chunk
// and 4-token tile of the batch, 64 16-bit words (one per lane), bit 15 - (4 j + i) = token i of
// the tile for the lane's neuron j.
constexpr int RELU_MASK_NPL = 4;
inline bool relu_mask_layer(int act, int pool, int K, int rec_shift, int x_dtype, int D) {
  return act == GL_ACT_RELU && (pool == GL_POOL_MEAN || pool == GL_POOL_SUM) && K == 8 && rec_shift == 0 &&
         !(x_dtype == GL_DTYPE_F32 && tiles_of_two(D));
}
inline size_t relu_mask_bytes(int G, int S, int B) {
  return (size_t)G * (size_t)ceil_div(S, 64 * RELU_MASK_NPL) * (size_t)ceil_div(B, 4) * 64 * 2;
}

// Max / top-k pooling backward as selection events (gl_max_bwd.hip): dW / db / dX of one token
// chunk [b0, b0 + Bc) from the chunk's token tiles, transposed coef / slots (c1t_kernel,
// events_transpose_kernel) and the row-major g_pre / selected slots.
struct MaxEvKArgs {
  const float4* xt;
  const int32_t* idx;
  const float* W;
  const float* bias;
  const int32_t* counts;
  const float* c1t;
  const int32_t* wint;
  const float* g_pre;
  const int32_t* winner;
  float* dW;
  float* db;
  float* dX;
  int D, G, S, cap, Bc, b0;
  int kpe;    // selected slots per (token, pool): 1 (max) or k (top-k mean)
  int rs;     // log2 slots per shared index record
  bool topk;  // coef = g_pre / min(n_g, kpe) (top-k mean) instead of g_pre
  int sps, gs;  // pool geometry (pool_base)
  int wbf;      // W and bias stored as bf16
};
int launch_max_events(int K, int act, const MaxEvKArgs& a, hipStream_t s);

// Launch trace (gl_trace_begin): record an event pair around one kernel launch.
void trace_before(hipStream_t s, int kernel_id);
void trace_after(hipStream_t s);
// hipLaunchKernelGGL wrapped by the launch trace; the stream is the launch's 5th argument
#define GL_LAUNCH(id, kernel, grid, block, lds, stream, ...)                        \
  do {                                                                             \
    ::gl::trace_before((stream), (id));                                            \
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);              \
    ::gl::trace_after((stream));                                                   \
  } while (0)

// Edge structure header (device buffer begins with it; arrays follow at the stated offsets).
struct EdgeHeader {
  uint32_t magic;        // GL_EDGE_MAGIC
  int32_t D, G, S, K;
  int32_t fw, us;        // features per range, slots per unit
  int32_t FR, P, U;      // feature ranges, pieces per group, units (= G * P)
  uint32_t nseg, n_edges;
  uint64_t off_seg_ptr, off_seg_unit, off_seg_begin, off_rec;  // byte offsets from the header
};
constexpr uint32_t GL_EDGE_MAGIC = 0x474c4531u;  // "GLE1"

}  // namespace gl
