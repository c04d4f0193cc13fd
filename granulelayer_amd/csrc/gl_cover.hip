// Cover-TopK support selection: for every envelope record of C = 16 gpb neurons sharing 64 input
// candidates, keep k candidates per 16-neuron row group (sparse_pooling/cover_topk16.py:1-24 and
// experimental/local_supports.py:209-222, 279-282, 294-375):
//   1. importance a[u, j] = sum over the valid neurons c of group u of W[u, c, j]^2, float64, added
//      in order c = 0..15;
//   2. TopK: the k largest a[u, j] per valid group, ties to the lower candidate position;
//   3. Cover repair: while some candidate j of the record is kept by no valid group, apply the swap
//      (u, d -> j) of smallest energy loss a[u, d] - a[u, j] over every uncovered j, valid group u and
//      kept donor d whose record count is >= 2 (ties: smallest j, then u; for the donor the smallest
//      a[u, d], then d).  Each swap covers one more candidate and uncovers none.
//
// One 64-lane wave per record, lane j = candidate j: the record's importances sit in LDS, each
// group's kept set is a 64-bit ballot mask, and every greedy step is a handful of wave-wide argmin
// reductions (DPP-free butterflies over (value, index) pairs: the lowest index wins ties, so the
// result does not depend on the reduction order).  Float64 throughout, integer bookkeeping; the
// output is bit-identical from run to run.
#include "gl_common.h"
#include "gl_internal.h"

namespace gl {

constexpr int COVER_S = 64;       // candidates per envelope record
constexpr int COVER_GPB_MAX = 16; // row groups per record (C <= 256)

struct CoverK {
  const float* W;
  const double* a;
  const int32_t* nvalid;
  const int32_t* cand;
  int R, gpb, k, repair;
  double* importance;
  int32_t* env;
  int32_t* rec_idx;
  float* W_out;
  int32_t* missing0;
  int32_t* swaps;
  double* loss;
  int32_t* status;
};

__device__ __forceinline__ double shfl_xor_d(double v, int m) {
  const long long b = __double_as_longlong(v);
  const int lo = __shfl_xor((int)(unsigned)b, m), hi = __shfl_xor((int)(b >> 32), m);
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// wave-wide minimum of (v, i) ordered by v, then the smaller i; every lane gets the result
__device__ __forceinline__ void wave_argmin(double& v, int& i) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const double ov = shfl_xor_d(v, m);
    const int oi = __shfl_xor(i, m);
    const bool take = ov < v || (ov == v && oi < i);
    v = take ? ov : v;
    i = take ? oi : i;
  }
}

__global__ void __launch_bounds__(64) cover_select_kernel(CoverK p) {
  __shared__ double A[COVER_GPB_MAX][COVER_S];
  const int r = blockIdx.x;
  const int j = threadIdx.x;
  const int gpb = p.gpb, C = 16 * gpb;
  int nv = p.nvalid[r];
  nv = nv < 0 ? 0 : (nv > C ? C : nv);
  const int m = (nv + 15) / 16;  // valid groups: a prefix of the record's groups
  const unsigned long long below = j ? (~0ull >> (64 - j)) : 0ull;  // candidates < j

  // 1. importances
  for (int u = 0; u < gpb; ++u) {
    const long long row = (long long)r * gpb + u;
    double acc;
    if (p.a) {
      acc = p.a[row * COVER_S + j];
    } else {
      const int nvu = nv - 16 * u;
      acc = 0.0;
      for (int c = 0; c < 16; ++c) {
        const double x = c < nvu ? (double)p.W[((long long)r * C + 16 * u + c) * COVER_S + j] : 0.0;
        acc = acc + x * x;  // x * x is exact in float64 (24-bit mantissas)
      }
    }
    A[u][j] = acc;
    if (p.importance) p.importance[row * COVER_S + j] = acc;
  }
  __syncthreads();

  // 2. top-k: the rank of candidate j in group u (larger first, the lower position on ties)
  unsigned long long X[COVER_GPB_MAX];
#pragma unroll
  for (int u = 0; u < COVER_GPB_MAX; ++u) {
    X[u] = 0ull;
    if (u >= gpb) continue;
    const double aj = A[u][j];
    int rank = 0;
    for (int i = 0; i < COVER_S; ++i) {
      const double ai = A[u][i];
      rank += (ai > aj || (ai == aj && i < j)) ? 1 : 0;
    }
    X[u] = __builtin_amdgcn_ballot_w64(rank < p.k);
  }

  // 3. coverage repair among the valid groups
  int miss0 = 0, nswap = 0, st = 0;
  double loss = 0.0;
  if (p.repair && m > 0) {
    if (m * p.k < COVER_S) {
      st = 1;  // infeasible: m k < 64 (the reference raises)
    } else {
      int cnt = 0;
#pragma unroll
      for (int u = 0; u < COVER_GPB_MAX; ++u) cnt += u < m ? (int)((X[u] >> j) & 1ull) : 0;
      miss0 = __builtin_popcountll(__builtin_amdgcn_ballot_w64(cnt == 0));
      const double inf = __builtin_inf();
      for (int round = 0; round < COVER_S; ++round) {
        if (__builtin_amdgcn_ballot_w64(cnt == 0) == 0ull) break;
        // cheapest removable donor of every valid group (a kept candidate counted >= 2 times)
        double dmin[COVER_GPB_MAX];
        int dstar[COVER_GPB_MAX];
#pragma unroll
        for (int u = 0; u < COVER_GPB_MAX; ++u) {
          dmin[u] = inf;
          dstar[u] = COVER_S;
          if (u >= m) continue;
          double v = (((X[u] >> j) & 1ull) && cnt >= 2) ? A[u][j] : inf;
          int i = j;
          wave_argmin(v, i);
          dmin[u] = v;
          dstar[u] = v < inf ? i : COVER_S;
        }
        // per uncovered candidate the best group (the smaller u on ties), then the best candidate
        double best = inf;
        int bu = COVER_GPB_MAX;
        if (cnt == 0) {
#pragma unroll
          for (int u = 0; u < COVER_GPB_MAX; ++u) {
            if (u >= m || !(dmin[u] < inf)) continue;
            const double cost = dmin[u] - A[u][j];
            if (cost < best) best = cost, bu = u;
          }
        }
        int key = j * COVER_GPB_MAX + bu;  // (j, u) order on equal costs
        wave_argmin(best, key);
        if (!(best < inf)) {
          st = 2;  // an uncovered candidate without a legal swap (cannot happen when m k >= 64)
          break;
        }
        const int jstar = key / COVER_GPB_MAX, ustar = key % COVER_GPB_MAX;
        int d = 0;
#pragma unroll
        for (int u = 0; u < COVER_GPB_MAX; ++u) d = u == ustar ? dstar[u] : d;
#pragma unroll
        for (int u = 0; u < COVER_GPB_MAX; ++u)
          X[u] = u == ustar ? (X[u] & ~(1ull << d)) | (1ull << jstar) : X[u];
        cnt += (j == jstar) - (j == d);
        loss += best;
        ++nswap;
      }
      if (st == 0 && __builtin_amdgcn_ballot_w64(cnt == 0) != 0ull) st = 2;
    }
  }
  if (j == 0) {
    if (p.missing0) p.missing0[r] = miss0;
    if (p.swaps) p.swaps[r] = nswap;
    if (p.loss) p.loss[r] = loss;
    if (p.status) p.status[r] = st;
  }

  // 4. outputs: kept positions ascending (padded groups: 0..k-1), their global inputs and weights
  const unsigned long long first_k = p.k >= 64 ? ~0ull : ((1ull << p.k) - 1ull);
#pragma unroll
  for (int u = 0; u < COVER_GPB_MAX; ++u) {
    if (u >= gpb) continue;
    const unsigned long long mask = u < m ? X[u] : first_k;
    if (!((mask >> j) & 1ull)) continue;
    const int pos = __builtin_popcountll(mask & below);
    const long long row = (long long)r * gpb + u;
    p.env[row * p.k + pos] = j;
    if (p.rec_idx) p.rec_idx[row * p.k + pos] = p.cand ? p.cand[(long long)r * COVER_S + j] : j;
    if (p.W_out) {
      const int nvu = nv - 16 * u;
      for (int c = 0; c < 16; ++c) {
        const long long n = (long long)r * C + 16 * u + c;
        p.W_out[n * p.k + pos] = c < nvu && p.W ? p.W[n * COVER_S + j] : 0.f;
      }
    }
  }
}

}  // namespace gl

using namespace gl;

extern "C" int gl_cover_select(const GlCoverArgs* a, void* stream) {
  if (!a || !a->nvalid || !a->env) return GL_ERR_ARG;
  if (!a->W && !a->a) return GL_ERR_ARG;
  if (a->R < 1 || a->gpb < 1 || a->gpb > COVER_GPB_MAX || a->k < 1 || a->k > COVER_S) return GL_ERR_ARG;
  if (a->W_out && !a->W) return GL_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  const CoverK k{a->W, a->a, a->nvalid, a->cand, a->R, a->gpb, a->k, a->repair ? 1 : 0, a->importance, a->env,
                 a->rec_idx, a->W_out, a->missing0, a->swaps, a->loss, a->status};
  GL_LAUNCH(GL_KERNEL_COVER, cover_select_kernel, dim3((unsigned)a->R), dim3(64), 0, s, k);
  GL_CHECK_LAUNCH();
  return 0;
}
