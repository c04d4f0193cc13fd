/*
 * granulelayer_amd -- C ABI of the MI355X (gfx950) sparse projection -> activation -> pool path.
 *
 * One layer: H neurons in G pools ("groups") of S padded slots; slot s of group g is a valid
 * neuron iff s < counts[g].  Every neuron owns a fan-in record of K input indices (the
 * reference's "Mode A", sparse_pooling/layout.py:1-34, SparseLayout(shared_indices=False)):
 *
 *   z[b,n]   = sum_k X[b, idx[n,k]] * W[n,k] + bias[n]
 *   pre[b,g] = scale_g * sum_{s < counts[g]} act(z[b, g*S+s])     scale_g = 1/counts[g] (mean) | 1 (sum)
 *
 * Conventions (the same as the reference's native ABI, sparse_pooling/backends/cuda/runtime.py:34-44):
 *   - every entry point returns 0 on success, a negative GL_ERR_* code when the library refuses
 *     the arguments, or a positive hipError_t when a launch failed;
 *   - the caller owns every buffer (inputs, outputs and workspace); the library never allocates
 *     device memory; sizes of workspaces come from the *_workspace / gl_edges_size queries;
 *   - work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the default stream) on
 *     the current HIP device; no host synchronisation happens inside any entry point;
 *   - all reductions have a fixed owner and order: repeated calls give bitwise-identical results.
 *     No floating-point atomics are used anywhere.
 */
#ifndef GRANULELAYER_AMD_H
#define GRANULELAYER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GL_ABI_VERSION 13

enum {
  GL_OK = 0,
  GL_ERR_ARG = -1,          /* invalid argument, shape or null pointer */
  GL_ERR_UNSUPPORTED = -2,  /* valid request this build does not implement (e.g. K not in {8,16}) */
  GL_ERR_WORKSPACE = -3,    /* workspace / output buffer smaller than required */
  GL_ERR_LDS = -4,          /* a kernel's LDS working set exceeds the device's LDS */
  GL_ERR_EDGES = -5,        /* edge structure built for a different layer shape */
  GL_ERR_DEVICE = -7,       /* no current HIP device or attribute query failed */
  GL_ERR_SCRATCH = -8       /* gl_fwd_static: one token tile of this layer exceeds the static scratch */
};
/* Largest input width D: the reference's int16 indices allow 32767 (sparse_pooling/layout.py:57-58).
 * D <= 4096 stages two token tiles in LDS, D <= 10112 one; wider layers gather X from the token
 * tiles in global memory (same results). */
#define GL_MAX_INPUTS 65536
/* neuron activation: identity, relu, exact (erf) GELU 0.5 z (1 + erf(z / sqrt 2)) (the reference's
 * ACTIVATIONS and _act / _dact, sparse_pooling/config.py:33, kernels/triton_fused.py:29-45) */
enum { GL_ACT_IDENTITY = 0, GL_ACT_RELU = 1, GL_ACT_GELU = 2 };
/* max: pytorch_reference.py:61-67 (winner = first maximum of act(z) over the pool's valid
 * slots), merged as kernels/ops.py:189-195; top-k mean: pytorch_reference.py:68-77 (the k largest
 * raw z, ties to the smaller slot, mean of act(z) over min(n_g, k) of them), ops.py:212-228 */
/* smooth operators (pytorch_reference.py:80-100), parameter in pool_param: LogMeanExp
 * pre = tau (logsumexp(a / tau) - log n_g) (tau = temperature); power mean (relu activations only)
 * pre = (mean a^p)^(1/p); softmax-weighted pre = sum softmax(beta a) a (beta) */
enum { GL_POOL_MEAN = 0, GL_POOL_SUM = 1, GL_POOL_MAX = 2, GL_POOL_TOPK_MEAN = 3, GL_POOL_LME = 4,
       GL_POOL_POWER = 5, GL_POOL_SOFTMAX = 6 };
enum { GL_DTYPE_F32 = 0, GL_DTYPE_BF16 = 1 };

/* Forward arguments.  Replaces the reference's FwdArgs + sp_fwd
 * (sparse_pooling/kernels/cuda/sparse_pool_fwd.cuh:23-38, sparse_pool.cu:12-23, mirrored in
 * backends/cuda/runtime.py:48-60) for the Mode-A path that the reference runs on Triton
 * (kernels/ops.py:104-154 fused_forward_states + :182-199 merge_finalize). */
typedef struct GlFwdArgs {
  const void* X;          /* [B, D] input, row stride sxb elements, dtype x_dtype */
  int64_t sxb;
  int32_t x_dtype;        /* GL_DTYPE_F32 | GL_DTYPE_BF16 */
  int32_t B, D, G, S, K;  /* tokens, inputs, groups, padded slots per group, fan-in (8 | 16) */
  int32_t act, pool;      /* GL_ACT_*, GL_POOL_* */
  int32_t topk;           /* GL_POOL_TOPK_MEAN: k, a power of two in [1, 64] (pools of <= 4096 slots) */
  int32_t rec_shift;      /* 0: every slot owns its index record; r in 1..4: 2^r consecutive slots share
                             one record (idx is [G*S >> r, K]; S a multiple of 2^r), e.g. r = 4 for the
                             K16 / C16 records of Cover-TopK/16 (sparse_pooling/cover_topk16.py:1-12) */
  int32_t sps, gs;        /* pool geometry.  sps <= 1: the G pools are the groups (S slots each; gs
                             0 or S).  sps > 1: two-level pooling's level-1 shards
                             (sparse_pooling/kernels/ops.py:45-56): the G pools are the sps shards of
                             G / sps groups of gs slots, pool u pooling slots
                             [(u % sps) * S, (u % sps) * S + counts[u]) of group u / sps, with
                             (sps - 1) * S < gs <= sps * S; tensors below indexed by neuron then have
                             G / sps * gs rows instead of G*S, and rec_shift must be 0 */
  const int32_t* idx;     /* [G*S >> rec_shift, K] input indices in [0, D) */
  const void* W;          /* [G*S, K], dtype w_dtype (4-byte aligned) */
  const void* bias;       /* [G*S], dtype w_dtype */
  const int32_t* counts;  /* [G] valid neurons per pool, 1 <= counts[g] <= S (and inside its group) */
  const uint32_t* sched;  /* gather schedule from gl_sched_build_host (K = 8), or NULL */
  const uint32_t* win;    /* [G] first input of each pool's window (gl_window_build_host), or NULL */
  int32_t win_width;      /* widest pool window; the kernels stage only the windows when narrow */
  float* pre;             /* out [B, G]: pooled value before the (identity) out-activation */
  int32_t* winner;        /* out [B, G, KPE] or NULL: the selected pool-local slots, KPE = 1 for
                             GL_POOL_MAX (the reference's "winner", ops.py:192-195), k for
                             GL_POOL_TOPK_MEAN ("topk_slot", best first, -1 past min(n_g, k)) */
  float pool_param;       /* GL_POOL_LME: temperature > 0; GL_POOL_POWER: p >= 1; GL_POOL_SOFTMAX: beta > 0 */
  float* lse;             /* out [B, G] or NULL: GL_POOL_LME / GL_POOL_SOFTMAX, the base-2 log-normaliser
                             L2 = log2 sum 2^(a * scale), scale = log2(e) / tau or log2(e) * beta (the
                             reference's "L2" statistic, kernels/ops.py:201-209) */
  void* ws;               /* workspace of gl_fwd_workspace() bytes */
  size_t ws_bytes;
  size_t part_budget;     /* bytes of per-chunk partial results one pass may hold (0: 8 GiB).  The
                             forward runs over token chunks whose partials fit it, so the workspace
                             stays bounded as B grows (the reference keeps its split states within
                             workspace_budget, sparse_pooling/kernels/ops.py:82-98) */
  int32_t w_dtype;        /* W and bias: GL_DTYPE_F32, or GL_DTYPE_BF16 read and widened in the kernels
                             (the reference's kernels load W in its stored dtype and widen it,
                             sparse_pooling/kernels/triton_fused.py:257) */
  void* relu_mask;        /* out or NULL: the ReLU bit (z > 0) of every (token, neuron), in the kernels'
                             own order, for GlBwdArgs.relu_mask; gl_fwd_mask_bytes() bytes.  Only for
                             the layers that query gives a non-zero size (GL_ACT_RELU with
                             GL_POOL_MEAN / GL_POOL_SUM, K = 8, rec_shift 0, 4-token X tiles).  The
                             reference keeps no such statistic: its backward recomputes z
                             (sparse_pooling/kernels/triton_fused.py:364-374); 1/32 of the [B, N]
                             hidden tensor's bytes buys the backward's dW pass that recompute */
} GlFwdArgs;

/* Backward arguments.  Replaces the reference's BwdArgs + sp_bwd (sparse_pool_bwd.cuh:45-66,
 * sparse_pool.cu:33-43, runtime.py:70-84) for the Mode-A path the reference runs on Triton
 * (autograd.py:275-300 _triton_backward, kernels/ops.py:242-278). */
typedef struct GlBwdArgs {
  const void* X;
  int64_t sxb;
  int32_t x_dtype;
  int32_t B, D, G, S, K;
  int32_t act, pool;
  int32_t topk;           /* as GlFwdArgs.topk */
  int32_t rec_shift;      /* as GlFwdArgs.rec_shift */
  int32_t sps, gs;        /* as GlFwdArgs.sps / gs */
  const int32_t* idx;
  const void* W;          /* as GlFwdArgs.W / bias (dtype w_dtype) */
  const void* bias;
  const int32_t* counts;
  const uint32_t* sched;  /* gather schedule from gl_sched_build_host (K = 8), or NULL */
  const uint32_t* win;    /* as GlFwdArgs.win / win_width */
  int32_t win_width;
  const float* g_pre;     /* [B, G] dL/dpre (fp32) */
  const int32_t* winner;  /* [B, G, KPE] the forward's selected slots: required for GL_POOL_MAX and
                             GL_POOL_TOPK_MEAN, NULL otherwise */
  float pool_param;       /* as GlFwdArgs.pool_param */
  const float* pre;       /* [B, G] the forward's pooled values: required for GL_POOL_POWER, GL_POOL_SOFTMAX
                             and (without lse) GL_POOL_LME */
  const float* lse;       /* [B, G] the forward's L2: required for GL_POOL_SOFTMAX; GL_POOL_LME recovers it
                             from pre when NULL (kernels/ops.py:251-254) */
  float* dW;              /* [G*S, K] ACCUMULATED (+=), e.g. W.main_grad; padded slots untouched */
  float* db;              /* [G*S] ACCUMULATED (+=) */
  float* dX;              /* out [B, D] fp32, overwritten */
  const void* edges;      /* input-major edge structure from gl_edges_build() for this idx/counts */
  size_t edges_bytes;
  void* ws;               /* workspace of gl_bwd_workspace() bytes */
  size_t ws_bytes;
  size_t dz_budget;       /* smooth pools (GL_POOL_LME / POWER / SOFTMAX): bytes of the per-neuron dz
                             of one backward token chunk, [G*S, chunk] fp32 (0: 8 GiB).  Chunks are of
                             64 to 1024 tokens, at least 64 whatever the budget; larger chunks run
                             fewer recompute and dX passes per token (the workspace query includes
                             it).  dW / db sum over the chunks, so their rounding depends on it */
  int32_t w_dtype;        /* as GlFwdArgs.w_dtype; dW and db are fp32 whatever it is */
  const void* relu_mask;  /* or NULL: the bits gl_fwd wrote into GlFwdArgs.relu_mask for the same X,
                             idx, W, bias, counts, sched and B; the dW pass then reads them instead of
                             recomputing z (results identical bit for bit) */
} GlBwdArgs;

/* Input-major (transposed) edge list of a layer, built once per index tensor.  It has no
 * reference counterpart: the reference's Mode-A dX is an fp32 atomic scatter
 * (sparse_pooling/kernels/triton_fused.py:442-445); this structure turns it into a
 * deterministic segmented reduction (the fixed-owner pattern of kernels/cuda/sg_det.cu:1-46). */
typedef struct GlEdgeArgs {
  const int32_t* idx;     /* [G*S >> rec_shift, K] */
  const int32_t* counts;
  int32_t D, G, S, K;
  int32_t rec_shift;      /* as GlFwdArgs.rec_shift */
  int32_t sps, gs;        /* as GlFwdArgs.sps / gs */
  void* edges;            /* out, gl_edges_size() bytes */
  size_t edges_bytes;
  void* ws;               /* scratch, gl_edges_size() bytes */
  size_t ws_bytes;
} GlEdgeArgs;

/* Fused AdamW step.  Replaces the Triton _adamw_kernel launch of FusedAdamW.step
 * (sparse_pooling/optim.py:26-64, 116-123) for fp32 parameters (HAS_MASTER = STOCH = False):
 *   m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g^2;  upd = (m/bc1) / (sqrt(v/bc2) + eps)
 *   p = p (1 - lr wd) - lr upd;  g = 0 (fused zero_grad) */
typedef struct GlAdamArgs {
  void* p;                /* parameters, fp32 or bf16 (p_dtype) */
  float* g;               /* fp32 gradient (main_grad), zeroed */
  void* m;                /* fp32 or bf16 (moments_dtype) */
  void* v;
  int64_t n;
  int32_t moments_dtype;  /* GL_DTYPE_F32 | GL_DTYPE_BF16 */
  float lr, beta1, beta2, eps, weight_decay, bc1, bc2;
  int32_t p_dtype;        /* GL_DTYPE_F32 | GL_DTYPE_BF16 */
  int32_t stochastic;     /* bf16 p without master: 1 = stochastic rounding (optim.py:59-62), 0 = nearest even */
  float* master;          /* bf16 p: fp32 master copy the update runs on (then p = nearest-even bf16 of it,
                             optim.py:54-56), or NULL */
  uint64_t seed;          /* stochastic rounding: element i adds the low 16 bits of Triton's
                             tl.randint(seed, i) (Philox-4x32-10) below the bf16 cut, then truncates */
} GlAdamArgs;

/* Cover-TopK support selection of an envelope (one-time preprocessing of CoverTopK16Layer).
 * Replaces local_supports.feature_importance / topk_select / cover_repair
 * (sparse_pooling/experimental/local_supports.py:209-222, 279-282, 294-375) as used by
 * CoverTopK16Layer.from_envelope (sparse_pooling/cover_topk16.py:80-146).  R envelope records of
 * C = 16 gpb neurons share 64 candidate inputs each; the valid neurons of a record are a prefix.
 * Per 16-neuron row group u: importance a[u, j] = sum over its valid neurons of W^2 (float64, in
 * neuron order); the k largest (ties to the lower position); with repair, every candidate of a
 * record is then kept by at least one valid group through greedy minimum-energy-loss swaps. */
typedef struct GlCoverArgs {
  const float* W;         /* [R * C, 64] envelope weights, or NULL when a is given */
  const double* a;        /* [R * gpb, 64] importances to select from, or NULL (computed from W) */
  const int32_t* nvalid;  /* [R] valid neurons of each record (0..C) */
  const int32_t* cand;    /* [R, 64] global input of each candidate, or NULL (rec_idx gets positions) */
  int32_t R, gpb, k;      /* records, row groups per record (1..16), kept candidates per group (1..64) */
  int32_t repair;         /* 1: Cover-TopK (coverage repair after TopK), 0: TopK only */
  double* importance;     /* out [R * gpb, 64] or NULL */
  int32_t* env;           /* out [R * gpb, k] kept positions, ascending (groups with no valid neuron: 0..k-1) */
  int32_t* rec_idx;       /* out [R * gpb, k] cand[record, env] or NULL */
  float* W_out;           /* out [R * C, k] every neuron's weights at its group's kept positions (0 for
                             padded neurons), or NULL */
  int32_t* missing0;      /* out [R] candidates kept by no valid group after TopK, or NULL */
  int32_t* swaps;         /* out [R] repair swaps, or NULL */
  double* loss;           /* out [R] energy loss of the swaps (float64, in swap order), or NULL */
  int32_t* status;        /* out [R] 0 ok, 1 infeasible record (valid groups * k < 64: nothing repaired),
                             or NULL */
} GlCoverArgs;

int gl_cover_select(const GlCoverArgs* a, void* stream);

/* ABI identity: version and struct layouts (sizeof, then every field offset in declaration
 * order) so a binding can refuse a mismatched library.  Replaces sp_abi_version /
 * sp_struct_layout (sparse_pooling/kernels/cuda/abi.cu:17-62, checked in runtime.py:103-120).
 * which: 0 GlFwdArgs, 1 GlBwdArgs, 2 GlEdgeArgs, 3 GlAdamArgs, 4 GlCoverArgs.  Returns the number of values
 * written (or needed, when n is too small), negative on an unknown struct. */
int gl_abi_version(void);
int gl_struct_layout(int which, long long* out, int n);
const char* gl_error_string(int code);

/* Forward.  gl_fwd_workspace writes the workspace size for these arguments to *bytes. */
int gl_fwd_workspace(const GlFwdArgs* a, size_t* bytes);
int gl_fwd(const GlFwdArgs* a, void* stream);
/* Bytes of GlFwdArgs.relu_mask for these arguments, 0 when the layer has no ReLU bits (then
 * relu_mask must be NULL).  No counterpart in the reference (whose backward recomputes z,
 * sparse_pooling/kernels/triton_fused.py:364-374). */
int gl_fwd_mask_bytes(const GlFwdArgs* a, size_t* bytes);

/* Forward that allocates nothing and takes no workspace.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The token tiles and partial results live in a
 * library-owned static device array of GL_FWD_STATIC_SCRATCH_BYTES per GPU (held from the first
 * call on that GPU until the process ends); a->ws, a->ws_bytes are ignored.  The forward runs as
 * many token passes as the array needs, with the results of gl_fwd; layers whose partials for one
 * 4-token tile exceed the array are refused with GL_ERR_SCRATCH.  Every call on a GPU shares that
 * GPU's array.  Outside graph capture, calls on different streams of one GPU are ordered by a
 * per-device "last use" event (each call's launches wait for the previous call's); under graph
 * capture the caller's graph must order the calls that share a GPU, or they race.  Nothing in it
 * needs zeroing between calls. */
#define GL_FWD_STATIC_SCRATCH_BYTES (64u << 20)
int gl_fwd_static(const GlFwdArgs* a, void* stream);

/* Edge structure: sizes (output and scratch) for a layer shape, then the build. */
int gl_edges_size(const GlEdgeArgs* a, size_t* edges_bytes, size_t* ws_bytes);
int gl_edges_build(const GlEdgeArgs* a, void* stream);

/* Backward: dW/db accumulated, dX written.  Recomputes z (nothing of size [B, H] is saved by
 * the forward).  gl_bwd_workspace writes the workspace size to *bytes. */
int gl_bwd_workspace(const GlBwdArgs* a, size_t* bytes);
int gl_bwd(const GlBwdArgs* a, void* stream);

/* Fused AdamW (in place). */
int gl_adam(const GlAdamArgs* a, void* stream);

/* Gather schedule of the forward and dW kernels (K = 8 only), built on the HOST once per index
 * tensor from host copies of idx [G*S, 8] and counts [G] (rec_shift 0); upload the result and pass it as
 * GlFwdArgs.sched / GlBwdArgs.sched.  It reorders, within windows of 128 slots, which neurons
 * share a 16-lane LDS gather and the order of each neuron's 8 edges, so the kernels' 16-byte LDS
 * reads hit distinct banks more often; results are unchanged up to fp32 summation order.  No
 * reference counterpart (the reference's Triton Mode-A kernels gather from global memory,
 * sparse_pooling/kernels/triton_fused.py:253-264).  threads <= 0: one per hardware thread. */
int gl_sched_size(int32_t G, int32_t S, int32_t K, size_t* bytes);
int gl_sched_build_host(const int32_t* idx, const int32_t* counts, int32_t D, int32_t G, int32_t S, int32_t sps,
                        int32_t gs, int32_t K, uint32_t* sched, int32_t threads);

/* The same schedule built on the GPU from device copies of idx and counts (one lane per 128-slot
 * window, the host builder's code), bit-identical to gl_sched_build_host; enqueued on stream. */
int gl_sched_build(const int32_t* idx, const int32_t* counts, int32_t D, int32_t G, int32_t S, int32_t sps,
                   int32_t gs, int32_t K, uint32_t* sched, void* stream);

/* Per-pool input windows, built on the HOST once per index tensor: lo[g] = the smallest input
 * index of pool g's valid neurons, *width = the widest window (largest - smallest + 1) over all
 * pools.  Pass lo as GlFwdArgs.win / GlBwdArgs.win and *width as win_width: when every workgroup's
 * pools fit (pools per workgroup x width rounded up to 64 <= 1024 inputs, and fewer than D) the
 * forward and dW kernels stage only those windows of X in LDS, 16 tokens per stage instead of 4.
 * Results are unchanged (same arithmetic, same order).  No reference counterpart in Mode A
 * (the reference stages per-supergroup feature sets in its Mode-B grouped kernels,
 * sparse_pooling/supergroups.py:1-40, kernels/cuda/sparse_pool_sg.cuh). */
int gl_window_build_host(const int32_t* idx, const int32_t* counts, int32_t D, int32_t G, int32_t S, int32_t sps,
                         int32_t gs, int32_t K, int32_t rec_shift, uint32_t* lo, int32_t* width);
/* The same windows built on the GPU from device copies (lo [G] and *width in device memory). */
int gl_window_build(const int32_t* idx, const int32_t* counts, int32_t D, int32_t G, int32_t S, int32_t sps,
                    int32_t gs, int32_t K, int32_t rec_shift, uint32_t* lo, int32_t* width, void* stream);

/* Kernel ids reported by the trace below. */
enum {
  GL_KERNEL_TILE_X = 1, GL_KERNEL_FWD = 2, GL_KERNEL_FWD_FINALIZE = 3, GL_KERNEL_C1T = 4, GL_KERNEL_BWD_W = 5,
  GL_KERNEL_DX = 6, GL_KERNEL_DX_REDUCE = 7, GL_KERNEL_ADAM = 8, GL_KERNEL_EDGES = 9,
  GL_KERNEL_FWD_WIN = 10, GL_KERNEL_BWD_W_WIN = 11, /* forward / dW with pool-window staging */
  GL_KERNEL_MAX_EV_DW = 12, GL_KERNEL_MAX_EV_DX = 13, /* max-pooling backward: winner events */
  GL_KERNEL_COVER = 14,                                /* Cover-TopK support selection */
  GL_KERNEL_SCHED = 15,                                /* gather schedule / pool windows on the GPU */
  GL_KERNEL_DX_DENSE = 16,                             /* dX of the smooth pools from per-neuron dz */
  GL_KERNEL_DX_DMA = 17                                /* dX of 256-token slices, short segments */
};

/* Launch trace for benchmarks and tests (process-wide, not for concurrent callers): after
 * gl_trace_begin, the i-th kernel launch of the library records events[2i] before and
 * events[2i+1] after itself on its stream and stores its GL_KERNEL_* id in kernel_ids[i],
 * for up to n_pairs launches; gl_trace_end stops recording and returns the number of launches
 * recorded.  events are hipEvent_t handles owned by the caller.  Replaces the reference's
 * PHASE_EVENTS hook (sparse_pooling/backends/cuda/runtime.py:131-148). */
int gl_trace_begin(void** events, int32_t* kernel_ids, int n_pairs);
int gl_trace_end(void);

#ifdef __cplusplus
}
#endif

#endif /* GRANULELAYER_AMD_H */
