// Input-major edge structure of the dX kernel, built once per index tensor.
//
// Edges (n, k) of valid slots are grouped into units u = (group g, piece of US slots) and
// ordered by the key (F = d / FW, u, d % FW, edge id).  Every unit is processed by one
// workgroup that sorts its own edges by (d, edge id) in LDS (bitonic, deterministic); the
// per-(F, u) counts are prefix-summed in F-major order to give each (F, u) run its global
// position.  Integer arithmetic only, no atomics on global memory: the output is bit-identical
// from run to run and to the numpy specification oracle/oracle.py:xedges.
#include "gl_common.h"
#include "gl_internal.h"

namespace gl {

void edge_layout(int D, int G, int S, int K, EdgeHeader* h, size_t* total);

constexpr int EB_THREADS = 512;

// slots of unit u that are valid: [s0, s1) of pool *g, whose first neuron is *nb
__device__ __forceinline__ void unit_slots(int u, int P, int S, int sps, int gs, const int32_t* counts, int* g,
                                           int* s0, int* s1, long long* nb) {
  *g = u / P;
  const int piece = u % P;
  *s0 = piece * US;
  *nb = pool_base(*g, S, sps, gs);
  const int ext = pool_ext(*g, S, sps, gs);
  int e = *s0 + US;
  if (e > ext) e = ext;
  const int n_g = counts[*g];
  if (e > n_g) e = n_g;
  *s1 = e < *s0 ? *s0 : e;
}

// cnt[F * U + u] = number of edges of unit u whose feature lies in range F (packed with the
// non-empty flag in the high 32 bits, for the segment count).
__global__ void __launch_bounds__(EB_THREADS) edges_count_kernel(const int32_t* __restrict__ idx,
                                                                 const int32_t* __restrict__ counts, int D, int S, int K,
                                                                 int rs, int sps, int gs, int P, int U, int FR,
                                                                 unsigned long long* __restrict__ cnt) {
  extern __shared__ unsigned hist[];
  const int u = blockIdx.x;
  int g, s0, s1;
  long long nb;
  unit_slots(u, P, S, sps, gs, counts, &g, &s0, &s1, &nb);
  for (int f = threadIdx.x; f < FR; f += blockDim.x) hist[f] = 0;
  __syncthreads();
  const long long n0 = nb + s0;
  const int ne = (s1 - s0) * K;
  for (int i = threadIdx.x; i < ne; i += blockDim.x) {
    int d = rec_index(idx, n0 + i / K, i % K, K, rs);
    d = d < 0 ? 0 : (d >= D ? D - 1 : d);
    atomicAdd(&hist[d / FW], 1u);
  }
  __syncthreads();
  for (int f = threadIdx.x; f < FR; f += blockDim.x) {
    const unsigned c = hist[f];
    cnt[(long long)f * U + u] = (unsigned long long)c | ((unsigned long long)(c > 0) << 32);
  }
}

// ---- exclusive scan of packed 64-bit counters (deterministic, three passes) ------------------
constexpr int SCAN_PER_THREAD = 8;
constexpr int SCAN_BLOCK = 256 * SCAN_PER_THREAD;

__global__ void __launch_bounds__(256) scan_local_kernel(unsigned long long* __restrict__ v, long long n,
                                                         unsigned long long* __restrict__ block_sum) {
  __shared__ unsigned long long sh[256];
  const long long base = (long long)blockIdx.x * SCAN_BLOCK + threadIdx.x * SCAN_PER_THREAD;
  unsigned long long loc[SCAN_PER_THREAD];
  unsigned long long run = 0;
#pragma unroll
  for (int i = 0; i < SCAN_PER_THREAD; ++i) {
    const long long j = base + i;
    const unsigned long long x = j < n ? v[j] : 0ull;
    loc[i] = run;
    run += x;
  }
  sh[threadIdx.x] = run;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {  // Hillis-Steele inclusive scan of thread totals
    unsigned long long t = threadIdx.x >= off ? sh[threadIdx.x - off] : 0ull;
    __syncthreads();
    sh[threadIdx.x] += t;
    __syncthreads();
  }
  const unsigned long long excl = threadIdx.x ? sh[threadIdx.x - 1] : 0ull;
#pragma unroll
  for (int i = 0; i < SCAN_PER_THREAD; ++i) {
    const long long j = base + i;
    if (j < n) v[j] = loc[i] + excl;
  }
  if (threadIdx.x == 255) block_sum[blockIdx.x] = sh[255];
}

// single workgroup: exclusive scan of the block sums in place; total at block_sum[nb]
__global__ void __launch_bounds__(1024) scan_blocks_kernel(unsigned long long* __restrict__ bs, int nb) {
  __shared__ unsigned long long sh[1024];
  __shared__ unsigned long long carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < nb; base += 1024) {
    const int j = base + threadIdx.x;
    const unsigned long long x = j < nb ? bs[j] : 0ull;
    sh[threadIdx.x] = x;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      unsigned long long t = threadIdx.x >= off ? sh[threadIdx.x - off] : 0ull;
      __syncthreads();
      sh[threadIdx.x] += t;
      __syncthreads();
    }
    const unsigned long long c = carry;
    if (j < nb) bs[j] = c + sh[threadIdx.x] - x;
    __syncthreads();
    if (threadIdx.x == 1023) carry = c + sh[1023];
    __syncthreads();
  }
  if (threadIdx.x == 0) bs[nb] = carry;
}

__global__ void __launch_bounds__(256) scan_add_kernel(unsigned long long* __restrict__ v, long long n,
                                                       const unsigned long long* __restrict__ bs) {
  const long long j = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (j < n) v[j] += bs[j / SCAN_BLOCK];
}

// ---- per-unit sort + scatter -----------------------------------------------------------------
struct ScatterK {
  const int32_t* __restrict__ idx;
  const int32_t* __restrict__ counts;
  const unsigned long long* __restrict__ off;  // exclusive scan of cnt (low: edge offset, high: segment index)
  uint32_t* rec;
  int32_t* seg_unit;
  uint32_t* seg_begin;
  int D, S, K, P, U, FR, npow2;
  int rs;  // log2 slots per shared index record
  int sps, gs;  // pool geometry (pool_base)
};

__global__ void __launch_bounds__(EB_THREADS) edges_scatter_kernel(ScatterK p) {
  extern __shared__ unsigned long long keys[];  // npow2 keys, then FR local offsets (uint)
  unsigned* loc = reinterpret_cast<unsigned*>(keys + p.npow2);
  const int u = blockIdx.x;
  int g, s0, s1;
  long long nb;
  unit_slots(u, p.P, p.S, p.sps, p.gs, p.counts, &g, &s0, &s1, &nb);
  const long long n0 = nb + s0;
  const int ne = (s1 - s0) * p.K;
  for (int i = threadIdx.x; i < p.npow2; i += blockDim.x) {
    unsigned long long key = ~0ull;
    if (i < ne) {
      int d = rec_index(p.idx, n0 + i / p.K, i % p.K, p.K, p.rs);
      d = d < 0 ? 0 : (d >= p.D ? p.D - 1 : d);
      key = ((unsigned long long)(unsigned)d << 32) | (unsigned)i;
    }
    keys[i] = key;
  }
  for (int f = threadIdx.x; f < p.FR; f += blockDim.x) loc[f] = 0;
  __syncthreads();
  // bitonic sort, ascending
  for (int size = 2; size <= p.npow2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < p.npow2 / 2; i += blockDim.x) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool asc = (lo & size) == 0;
        const unsigned long long a = keys[lo], b = keys[hi];
        if ((a > b) == asc) {
          keys[lo] = b;
          keys[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  // first sorted position of every feature range present in this unit
  for (int i = threadIdx.x; i < ne; i += blockDim.x) {
    const int F = (int)(keys[i] >> 32) / FW;
    const int Fp = i > 0 ? (int)(keys[i - 1] >> 32) / FW : -1;
    if (F != Fp) loc[F] = (unsigned)i;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < ne; i += blockDim.x) {
    const unsigned long long key = keys[i];
    const int d = (int)(key >> 32);
    const int F = d / FW;
    const unsigned el = (unsigned)key;  // s_local * K + k
    const unsigned long long o = p.off[(long long)F * p.U + u];
    const unsigned pos = (unsigned)o + ((unsigned)i - loc[F]);
    const bool newf = (unsigned)i != loc[F] && (int)(keys[i - 1] >> 32) != d;
    p.rec[pos] = el * 4u | ((unsigned)(d % FW) << REC_F_SHIFT) | (newf ? REC_NEWF : 0u);
    if ((unsigned)i == loc[F]) {
      const unsigned seg = (unsigned)(o >> 32);
      p.seg_unit[seg] = u;
      p.seg_begin[seg] = (unsigned)o;
    }
  }
}

// seg_ptr[F] = segment index at (F, u = 0); seg_ptr[FR] = nseg; seg_begin[nseg] = E; header.
__global__ void edges_finish_kernel(const unsigned long long* __restrict__ off, const unsigned long long* __restrict__ total,
                                    int U, int FR, uint32_t* seg_ptr, uint32_t* seg_begin, EdgeHeader h,
                                    EdgeHeader* out_h) {
  const int F = blockIdx.x * blockDim.x + threadIdx.x;
  const unsigned long long tot = *total;
  if (F < FR) seg_ptr[F] = (uint32_t)(off[(long long)F * U] >> 32);
  if (F == 0) {
    seg_ptr[FR] = (uint32_t)(tot >> 32);
    seg_begin[tot >> 32] = (uint32_t)tot;
    h.nseg = (uint32_t)(tot >> 32);
    h.n_edges = (uint32_t)tot;
    *out_h = h;
  }
}

static int pow2_at_least(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

}  // namespace gl

using namespace gl;

extern "C" int gl_edges_size(const GlEdgeArgs* a, size_t* edges_bytes, size_t* ws_bytes) {
  if (!a || !edges_bytes || !ws_bytes) return GL_ERR_ARG;
  if (a->D < 1 || a->G < 1 || a->S < 1) return GL_ERR_ARG;
  if (a->K != 8 && a->K != 16) return GL_ERR_UNSUPPORTED;
  if ((long long)a->G * a->S * a->K >= (1LL << 32)) return GL_ERR_UNSUPPORTED;
  GL_TRY(check_rec_shift(a->rec_shift, a->S, nullptr));
  int32_t sps = a->sps, gs = a->gs;
  GL_TRY(check_geometry(a->G, a->S, &sps, &gs));
  if (sps > 1 && a->rec_shift > 0) return GL_ERR_UNSUPPORTED;
  EdgeHeader h;
  edge_layout(a->D, a->G, a->S, a->K, &h, edges_bytes);
  const long long n = (long long)h.FR * h.U;
  const long long nb = (n + SCAN_BLOCK - 1) / SCAN_BLOCK;
  *ws_bytes = (size_t)round_up(n * 8, 256) + (size_t)round_up((nb + 1) * 8, 256);
  return 0;
}

extern "C" int gl_edges_build(const GlEdgeArgs* a, void* stream) {
  if (!a || !a->idx || !a->counts || !a->edges || !a->ws) return GL_ERR_ARG;
  size_t eb = 0, wb = 0;
  GL_TRY(gl_edges_size(a, &eb, &wb));
  if (a->edges_bytes < eb || a->ws_bytes < wb) return GL_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  const int sps = a->sps > 1 ? a->sps : 1, gs = a->sps > 1 ? a->gs : a->S;  // checked by gl_edges_size
  EdgeHeader h;
  edge_layout(a->D, a->G, a->S, a->K, &h, &eb);
  h.nseg = 0;
  h.n_edges = 0;
  const long long n = (long long)h.FR * h.U;
  const long long nb = (n + SCAN_BLOCK - 1) / SCAN_BLOCK;
  unsigned long long* cnt = (unsigned long long*)a->ws;
  unsigned long long* bsum = (unsigned long long*)((char*)a->ws + round_up(n * 8, 256));
  char* e = (char*)a->edges;

  const size_t hist_lds = (size_t)h.FR * 4;
  if (hist_lds > max_lds_bytes()) return GL_ERR_LDS;
  GL_TRY(set_lds_limit((const void*)edges_count_kernel, hist_lds));
  GL_LAUNCH(GL_KERNEL_EDGES, edges_count_kernel, dim3((unsigned)h.U), dim3(EB_THREADS), hist_lds, s, a->idx, a->counts, a->D,
                     a->S, a->K, a->rec_shift, sps, gs, h.P, h.U, h.FR, cnt);
  GL_CHECK_LAUNCH();
  GL_LAUNCH(GL_KERNEL_EDGES, scan_local_kernel, dim3((unsigned)nb), dim3(256), 0, s, cnt, n, bsum);
  GL_CHECK_LAUNCH();
  GL_LAUNCH(GL_KERNEL_EDGES, scan_blocks_kernel, dim3(1), dim3(1024), 0, s, bsum, (int)nb);
  GL_CHECK_LAUNCH();
  GL_LAUNCH(GL_KERNEL_EDGES, scan_add_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, cnt, n,
                     (const unsigned long long*)bsum);
  GL_CHECK_LAUNCH();

  const int per_unit = (US < a->S ? US : a->S) * a->K;
  const int npow2 = pow2_at_least(per_unit);
  const size_t sort_lds = (size_t)npow2 * 8 + (size_t)h.FR * 4;
  if (sort_lds > max_lds_bytes()) return GL_ERR_LDS;
  GL_TRY(set_lds_limit((const void*)edges_scatter_kernel, sort_lds));
  ScatterK sk{a->idx, a->counts, cnt, (uint32_t*)(e + h.off_rec), (int32_t*)(e + h.off_seg_unit),
              (uint32_t*)(e + h.off_seg_begin), a->D, a->S, a->K, h.P, h.U, h.FR, npow2, a->rec_shift, sps, gs};
  GL_LAUNCH(GL_KERNEL_EDGES, edges_scatter_kernel, dim3((unsigned)h.U), dim3(EB_THREADS), sort_lds, s, sk);
  GL_CHECK_LAUNCH();
  GL_LAUNCH(GL_KERNEL_EDGES, edges_finish_kernel, dim3((unsigned)ceil_div(h.FR, 256)), dim3(256), 0, s,
                     (const unsigned long long*)cnt, (const unsigned long long*)(bsum + nb), h.U, h.FR,
                     (uint32_t*)(e + h.off_seg_ptr), (uint32_t*)(e + h.off_seg_begin), h, (EdgeHeader*)e);
  GL_CHECK_LAUNCH();
  return 0;
}
