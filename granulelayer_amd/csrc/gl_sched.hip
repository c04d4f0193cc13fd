// Gather schedule of the neuron-stationary kernels (forward and dW), built on the host once per
// index tensor.
//
// Those kernels read, per (neuron slot j, k), one 16-byte LDS entry X[d] (4 tokens) per lane with
// ds_read_b128.  The LDS serves a b128 read in passes of 16 lanes; a pass is conflict-free when
// its 16 lanes read 16 distinct 16-byte slots mod 16, i.e. distinct residues d mod 16.  With
// random indices a 16-lane group averages ~3 passes.  The schedule lowers that by choosing
//   * which 16 neurons of a window of 128 slots share a 16-lane group ("set"), so each set's
//     residue histogram is flat (greedy: neurons with the most repeated residue first, each to
//     the set whose sum of squared excess over 8 per residue grows least), and
//   * the order in which every neuron visits its K = 8 edges: round by round, a maximum matching
//     of the set's 16 lanes to distinct residues among their unused edges (augmenting paths,
//     residues with more remaining edges tried first); unmatched lanes take the edge whose
//     residue the round uses least.
// Both only reorder a pool's neurons and each neuron's terms, so the pooled sum and every
// gradient keep their value (fp32 rounding order aside).
//
// Record of lane l, neuron slot j of a chunk that starts at window w0 (chunk slots are multiples
// of 128): window w = w0 + j / 2, set = (j % 2) * 4 + l / 16, position = set * 16 + l % 16;
// sched[(g * nwin + w) * 128 + position] = s_local | k_0 << 7 | k_1 << 10 | ... | k_6 << 25, where
// s_local (0..127) is the slot within the window and k_0..k_6 the first seven edges in visiting
// order (k_7 = 28 - their sum).
#include <algorithm>
#include <thread>
#include <vector>

#include "gl_common.h"
#include "gl_internal.h"

namespace gl {
namespace {

constexpr int WIN = 128;
constexpr int SETS = WIN / 16;
constexpr int KS = 8;

// One window of 128 slots: the residues of its edges and the working arrays of the schedule, in one
// struct of narrow types.  The same code runs on the host (gl_sched_build_host, one struct per
// thread) and on the GPU (gl_sched_build, one struct per lane in LDS), so both builders give the
// same schedule bit for bit.  A slot is invalid (past the pool's n_g) when its res row is -1.
struct WinWork {
  int8_t res[WIN][KS];     // residue of edge k of slot p (-1: invalid slot)
  uint8_t order[WIN];      // balance: slots by most repeated residue, then slot
  uint8_t mxv[WIN];        // balance: multiplicity of slot p's most repeated residue
  uint8_t H[SETS][16];     // balance: residue counts of each set (<= 128)
  uint8_t members[SETS][16];
  uint8_t cnt[SETS];
  int8_t rem[16][KS];      // match: residue of each lane's unused edge k (-1 = used)
  uint8_t kperm[16][KS];   // match: visiting order
  uint32_t cand[16];       // matcher: residues of lane l's unused edges
  int8_t ord[16];          // matcher: residues, most remaining edges first
  int8_t owner[16];        // matcher: lane holding residue r (-1: free)
  uint8_t deg[16], ndist[16], lord[16], used[16];
  int8_t lane_res[16];
  int8_t st_lane[17], st_pos[17], st_tried[17];  // matcher: depth-first stack
  uint8_t pad[7];          // 2036 bytes: an odd number of dwords, so lanes' structs start on different banks
};

// stable insertion sort of v[0..n) by key (larger first when desc): the order std::stable_sort
// gives for the same comparator
template <typename T, typename KeyF>
__host__ __device__ inline void stable_sort_by(T* v, int n, KeyF key, bool desc) {
  for (int i = 1; i < n; ++i) {
    const T x = v[i];
    const int kx = key(x);
    int j = i - 1;
    while (j >= 0 && (desc ? key(v[j]) < kx : key(v[j]) > kx)) {
      v[j + 1] = v[j];
      --j;
    }
    v[j + 1] = x;
  }
}

// slot p's distinct residues in ascending order (bit r of the mask) and multiplicity of residue r
__host__ __device__ inline unsigned slot_mask(const WinWork& W, int p) {
  unsigned m = 0u;
  for (int k = 0; k < KS; ++k)
    if (W.res[p][k] >= 0) m |= 1u << W.res[p][k];
  return m;
}
__host__ __device__ inline int slot_mult(const WinWork& W, int p, int r) {
  int c = 0;
  for (int k = 0; k < KS; ++k) c += W.res[p][k] == r;
  return c;
}

// greedy balance: slots with the most repeated residue first; each goes to the set (with room)
// whose sum over residues of (count - 8)^2 for counts above 8 grows least (ties: lower set)
__host__ __device__ inline void balance(WinWork& W) {
  for (int p = 0; p < WIN; ++p) {
    W.order[p] = (uint8_t)p;
    int mx = 0;
    for (int k = 0; k < KS; ++k)
      if (W.res[p][k] >= 0) {
        const int c = slot_mult(W, p, W.res[p][k]);
        mx = mx > c ? mx : c;
      }
    W.mxv[p] = (uint8_t)mx;
  }
  stable_sort_by(W.order, WIN, [&](uint8_t a) { return (int)W.mxv[a]; }, true);
  for (int set = 0; set < SETS; ++set) {
    W.cnt[set] = 0;
    for (int r = 0; r < 16; ++r) W.H[set][r] = 0;
  }
  for (int oi = 0; oi < WIN; ++oi) {
    const int p = W.order[oi];
    const unsigned m = slot_mask(W, p);  // the distinct residues of slot p, ascending
    int best = -1, best_cost = 0;
    for (int set = 0; set < SETS; ++set) {
      if (W.cnt[set] == 16) continue;
      int c = 0;
      for (unsigned b = m; b; b &= b - 1) {
        const int r = __builtin_ctz(b), h = slot_mult(W, p, r);
        const int before = W.H[set][r] - 8, after = before + h;
        c += (after > 0 ? after * after : 0) - (before > 0 ? before * before : 0);
      }
      if (best < 0 || c < best_cost) best = set, best_cost = c;
    }
    for (unsigned b = m; b; b &= b - 1) {
      const int r = __builtin_ctz(b);
      W.H[best][r] = (uint8_t)(W.H[best][r] + slot_mult(W, p, r));
    }
    W.members[best][W.cnt[best]++] = (uint8_t)p;
  }
}

// Kuhn's augmenting paths over 16 lanes and 16 residues; cand[l] = residues of lane l's unused
// edges, tried in the round's residue order (most remaining edges first).  Depth-first search with
// an explicit stack: frame f holds its lane, the next residue position to try and the residue it
// is trying; a free residue found at depth d gives every frame on the path its residue.
__host__ __device__ inline bool try_lane(WinWork& W, int l0) {
  uint32_t seen = 0;
  int d = 0;
  W.st_lane[0] = (int8_t)l0;
  W.st_pos[0] = 0;
  for (;;) {
    const int l = W.st_lane[d];
    bool pushed = false;
    while (W.st_pos[d] < 16) {
      const int r = W.ord[W.st_pos[d]];
      W.st_pos[d] = (int8_t)(W.st_pos[d] + 1);
      if (!((W.cand[l] >> r) & 1u) || ((seen >> r) & 1u)) continue;
      seen |= 1u << r;
      if (W.owner[r] < 0) {
        W.owner[r] = (int8_t)l;
        for (int f = d - 1; f >= 0; --f) W.owner[W.st_tried[f]] = W.st_lane[f];
        return true;
      }
      W.st_tried[d] = (int8_t)r;
      W.st_lane[d + 1] = W.owner[r];
      W.st_pos[d + 1] = 0;
      ++d;
      pushed = true;
      break;
    }
    if (pushed) continue;
    if (d == 0) return false;
    --d;  // the child found no augmenting path: continue this frame's residues
  }
}

// visiting order W.kperm[lane][round] of set `set`'s lanes; invalid lanes keep the identity
__host__ __device__ inline void match_set(WinWork& W, int set) {
  unsigned live = 0u;  // bit l: lane l's slot is valid
  for (int l = 0; l < 16; ++l) {
    const int p = W.members[set][l];
    if (W.res[p][0] >= 0) live |= 1u << l;
    for (int k = 0; k < KS; ++k) {
      W.rem[l][k] = (live >> l) & 1u ? W.res[p][k] : (int8_t)-1;
      W.kperm[l][k] = (uint8_t)k;
    }
  }
  for (int round = 0; round < KS; ++round) {
    for (int r = 0; r < 16; ++r) W.deg[r] = 0;
    for (int l = 0; l < 16; ++l) {
      unsigned c = 0u;
      for (int k = 0; k < KS; ++k)
        if (W.rem[l][k] >= 0) W.deg[W.rem[l][k]]++, c |= 1u << W.rem[l][k];
      W.cand[l] = c;
      W.ndist[l] = (uint8_t)__builtin_popcount(c);
    }
    for (int r = 0; r < 16; ++r) W.ord[r] = (int8_t)r, W.owner[r] = -1;
    stable_sort_by(W.ord, 16, [&](int8_t a) { return (int)W.deg[a]; }, true);
    for (int l = 0; l < 16; ++l) W.lord[l] = (uint8_t)l;
    stable_sort_by(W.lord, 16, [&](uint8_t a) { return (int)W.ndist[a]; }, false);
    for (int i = 0; i < 16; ++i) {
      const int l = W.lord[i];
      if (!((live >> l) & 1u)) continue;
      try_lane(W, l);
    }
    for (int l = 0; l < 16; ++l) W.lane_res[l] = -1, W.used[l] = 0;
    for (int r = 0; r < 16; ++r)
      if (W.owner[r] >= 0) W.lane_res[W.owner[r]] = (int8_t)r, W.used[r]++;
    for (int l = 0; l < 16; ++l) {  // unmatched lanes: the residue this round uses least
      if (!((live >> l) & 1u) || W.lane_res[l] >= 0) continue;
      int best = -1;
      for (int k = 0; k < KS; ++k) {
        const int r = W.rem[l][k];
        if (r < 0) continue;
        if (best < 0 || W.used[r] < W.used[best] ||
            (W.used[r] == W.used[best] && (W.deg[r] > W.deg[best] || (W.deg[r] == W.deg[best] && r < best))))
          best = r;
      }
      W.lane_res[l] = (int8_t)best;
      W.used[best]++;
    }
    for (int l = 0; l < 16; ++l) {
      if (!((live >> l) & 1u)) continue;
      for (int k = 0; k < KS; ++k)  // the lowest unused edge with that residue
        if (W.rem[l][k] == W.lane_res[l]) {
          W.kperm[l][round] = (uint8_t)k;
          W.rem[l][k] = -1;
          break;
        }
    }
  }
}

// slot p's residues (window w of group g)
__host__ __device__ inline void load_slot(WinWork& W, const int32_t* idx, int D, long long nb, int w, int n_g, int p) {
  const int s = w * WIN + p;
  const bool valid = s < n_g;
  for (int k = 0; k < KS; ++k) {
    int r = -1;
    if (valid) {
      int d = idx[(nb + s) * KS + k];
      d = d < 0 ? 0 : (d >= D ? D - 1 : d);
      r = d & 15;
    }
    W.res[p][k] = (int8_t)r;
  }
}

// the 128 records of one loaded window
__host__ __device__ inline void schedule_window(WinWork& W, uint32_t* out) {
  balance(W);
  for (int set = 0; set < SETS; ++set) {
    match_set(W, set);
    for (int l = 0; l < 16; ++l) {
      uint32_t rec = (uint32_t)W.members[set][l];
      for (int ks = 0; ks < KS - 1; ++ks) rec |= (uint32_t)W.kperm[l][ks] << (7 + 3 * ks);
      out[set * 16 + l] = rec;
    }
  }
}

void build_range(const int32_t* idx, const int32_t* counts, int D, int S, int sps, int gs, long long w_begin,
                 long long w_end, uint32_t* sched) {
  const int nwin = ceil_div(S, WIN);
  WinWork W;
  for (long long gw = w_begin; gw < w_end; ++gw) {
    const long long g = gw / nwin;
    const int w = (int)(gw % nwin);
    const int n_g = std::min(counts[g], pool_ext((int)g, S, sps, gs));
    const long long nb = pool_base((int)g, S, sps, gs);
    for (int p = 0; p < WIN; ++p) load_slot(W, idx, D, nb, w, n_g, p);
    schedule_window(W, sched + gw * WIN);
  }
}

// GPU builder: one window per lane, its working struct (2036 bytes) in the lane's private memory,
// 128 VGPRs so a SIMD runs 4 waves.  The walk is latency-bound, so waves count: the C2 layer's
// schedule took 1.45 s with the earlier per-lane arrays (a 16-bit histogram per slot, int locals:
// ~6 KB per lane), 0.72 s with the compact struct at 2 waves per SIMD and 0.54 s at 4; with the 64
// structs of a workgroup in LDS (one wave per CU) 2.3 s.
constexpr int SCHED_LANES = 64;
static_assert(sizeof(WinWork) == 2036, "WinWork: an odd number of dwords");
__global__ void __launch_bounds__(SCHED_LANES) __attribute__((amdgpu_waves_per_eu(4, 4)))
sched_build_kernel(const int32_t* __restrict__ idx, const int32_t* __restrict__ counts, int D, int S, int sps, int gs,
                   int nwin, long long nw, uint32_t* __restrict__ sched) {
  const long long gw = (long long)blockIdx.x * SCHED_LANES + threadIdx.x;
  if (gw >= nw) return;
  const long long g = gw / nwin;
  const int w = (int)(gw % nwin);
  const int ext = pool_ext((int)g, S, sps, gs);
  const int n_g = counts[g] < ext ? counts[g] : ext;
  const long long nb = pool_base((int)g, S, sps, gs);
  WinWork W;
  for (int p = 0; p < WIN; ++p) load_slot(W, idx, D, nb, w, n_g, p);
  schedule_window(W, sched + gw * WIN);
}

__global__ void fill_i32_kernel(int32_t* p, int n, int32_t v) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = v;
}

// GPU pool windows: one workgroup per pool, the smallest and largest index of its valid slots'
// records; the widest window by an integer atomic maximum (order-independent)
__global__ void __launch_bounds__(256) window_build_kernel(const int32_t* __restrict__ idx,
                                                           const int32_t* __restrict__ counts, int D, int S, int sps,
                                                           int gs, int K, int rs, uint32_t* __restrict__ lo,
                                                           int32_t* __restrict__ width) {
  __shared__ int smn[4], smx[4];
  const int g = blockIdx.x;
  const int ext = pool_ext(g, S, sps, gs);
  const int n_g = counts[g] < ext ? counts[g] : ext;
  const long long nb = pool_base(g, S, sps, gs);
  const long long r0 = nb >> rs;
  const long long r1 = n_g > 0 ? ((nb + n_g - 1) >> rs) + 1 : r0;
  int mn = D, mx = -1;
  for (long long e = r0 * K + threadIdx.x; e < r1 * K; e += blockDim.x) {
    int d = idx[e];
    d = d < 0 ? 0 : (d >= D ? D - 1 : d);
    mn = d < mn ? d : mn;
    mx = d > mx ? d : mx;
  }
  for (int o = 32; o > 0; o >>= 1) {
    const int a = __shfl_xor(mn, o), b = __shfl_xor(mx, o);
    mn = a < mn ? a : mn;
    mx = b > mx ? b : mx;
  }
  if ((threadIdx.x & 63) == 0) smn[threadIdx.x >> 6] = mn, smx[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 4; ++i) mn = smn[i] < mn ? smn[i] : mn, mx = smx[i] > mx ? smx[i] : mx;
    if (mx < 0) mn = mx = 0;
    lo[g] = (uint32_t)mn;
    atomicMax(width, mx - mn + 1);
  }
}

}  // namespace
}  // namespace gl

using namespace gl;

extern "C" int gl_sched_size(int32_t G, int32_t S, int32_t K, size_t* bytes) {
  if (!bytes || G < 1 || S < 1) return GL_ERR_ARG;
  if (K != 8) return GL_ERR_UNSUPPORTED;
  *bytes = (size_t)G * ceil_div(S, WIN) * WIN * sizeof(uint32_t);
  return 0;
}

extern "C" int gl_sched_build_host(const int32_t* idx, const int32_t* counts, int32_t D, int32_t G, int32_t S,
                                   int32_t sps, int32_t gs, int32_t K, uint32_t* sched, int32_t threads) {
  if (!idx || !counts || !sched || D < 1 || G < 1 || S < 1) return GL_ERR_ARG;
  GL_TRY(check_geometry(G, S, &sps, &gs));
  if (K != 8) return GL_ERR_UNSUPPORTED;
  const long long nw = (long long)G * ceil_div(S, WIN);
  int nt = threads > 0 ? threads : (int)std::thread::hardware_concurrency();
  if (nt < 1) nt = 1;
  if (nt > 256) nt = 256;
  if ((long long)nt > nw) nt = (int)nw;
  std::vector<std::thread> pool;
  for (int t = 0; t < nt; ++t) {
    const long long b = nw * t / nt, e = nw * (t + 1) / nt;
    pool.emplace_back(build_range, idx, counts, D, S, sps, gs, b, e, sched);
  }
  for (auto& th : pool) th.join();
  return 0;
}

// Per-pool input windows (no reference counterpart; the per-pool analogue of the reference's
// per-supergroup feature sets, sparse_pooling/supergroups.py:1-40): lo[g] = the smallest index
// of pool g's valid neurons, *width = max over pools of (largest - smallest + 1).  With narrow
// windows the forward and dW kernels stage only each pool's window of X in LDS.
extern "C" int gl_window_build_host(const int32_t* idx, const int32_t* counts, int32_t D, int32_t G, int32_t S,
                                    int32_t sps, int32_t gs, int32_t K, int32_t rec_shift, uint32_t* lo, int32_t* width) {
  if (!idx || !counts || !lo || !width || D < 1 || G < 1 || S < 1 || K < 1) return GL_ERR_ARG;
  if (rec_shift < 0 || rec_shift > 4 || S % (1 << rec_shift) != 0) return GL_ERR_ARG;
  GL_TRY(check_geometry(G, S, &sps, &gs));
  if (rec_shift > 0 && sps > 1) return GL_ERR_UNSUPPORTED;
  int32_t wmax = 0;
  for (int g = 0; g < G; ++g) {
    const int ext = pool_ext(g, S, sps, gs);
    const int n_g = counts[g] < ext ? counts[g] : ext;
    int32_t mn = D, mx = -1;
    // the records that hold the pool's valid slots [0, n_g): rows nb >> r .. (nb + n_g - 1) >> r
    const long long nb = pool_base(g, S, sps, gs);
    const long long r0 = nb >> rec_shift;
    const long long r1 = n_g > 0 ? ((nb + n_g - 1) >> rec_shift) + 1 : r0;
    for (long long e = r0 * K; e < r1 * K; ++e) {
      int32_t d = idx[e];
      d = d < 0 ? 0 : (d >= D ? D - 1 : d);
      mn = d < mn ? d : mn;
      mx = d > mx ? d : mx;
    }
    if (mx < 0) mn = mx = 0;
    lo[g] = (uint32_t)mn;
    wmax = mx - mn + 1 > wmax ? mx - mn + 1 : wmax;
  }
  *width = wmax;
  return 0;
}

extern "C" int gl_sched_build(const int32_t* idx, const int32_t* counts, int32_t D, int32_t G, int32_t S, int32_t sps,
                              int32_t gs, int32_t K, uint32_t* sched, void* stream) {
  if (!idx || !counts || !sched || D < 1 || G < 1 || S < 1) return GL_ERR_ARG;
  GL_TRY(check_geometry(G, S, &sps, &gs));
  if (K != 8) return GL_ERR_UNSUPPORTED;
  const long long nw = (long long)G * ceil_div(S, WIN);
  if (nw >= (1LL << 31)) return GL_ERR_UNSUPPORTED;
  GL_LAUNCH(GL_KERNEL_SCHED, sched_build_kernel, dim3((unsigned)ceil_div(nw, SCHED_LANES)), dim3(SCHED_LANES), 0,
            (hipStream_t)stream, idx,
            counts, D, S, sps, gs, ceil_div(S, WIN), nw, sched);
  GL_CHECK_LAUNCH();
  return 0;
}

extern "C" int gl_window_build(const int32_t* idx, const int32_t* counts, int32_t D, int32_t G, int32_t S, int32_t sps,
                               int32_t gs, int32_t K, int32_t rec_shift, uint32_t* lo, int32_t* width, void* stream) {
  if (!idx || !counts || !lo || !width || D < 1 || G < 1 || S < 1 || K < 1) return GL_ERR_ARG;
  if (rec_shift < 0 || rec_shift > 4 || S % (1 << rec_shift) != 0) return GL_ERR_ARG;
  GL_TRY(check_geometry(G, S, &sps, &gs));
  if (rec_shift > 0 && sps > 1) return GL_ERR_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  GL_LAUNCH(GL_KERNEL_SCHED, fill_i32_kernel, dim3(1), dim3(64), 0, s, width, 1, 0);
  GL_CHECK_LAUNCH();
  GL_LAUNCH(GL_KERNEL_SCHED, window_build_kernel, dim3((unsigned)G), dim3(256), 0, s, idx, counts, D, S, sps, gs, K,
            rec_shift, lo, width);
  GL_CHECK_LAUNCH();
  return 0;
}
