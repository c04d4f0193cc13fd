// LDS gather-rate probe (a measurement tool, not part of the layer's library): how many bytes per
// clock a CU's LDS delivers to ds_read_b128 / ds_read_b64 gathers whose lanes read given slots of
// a 64-KiB tile.  The forward and dW kernels gather 16-byte (4-token fp32) or 8-byte (4-token bf16,
// 2-token fp32) slots of random inputs; which lane-to-bank patterns run at which rate decides their
// gather schedule.  Built as its own shared library (libgl_lds_probe.so) and driven by
// `bench.py --lds-probe`, which writes the patterns and prints the table.
//
// One workgroup of 16 waves per CU.  Every wave reads the same 8 patterns (8 independent reads per
// loop iteration, one slot offset per lane and pattern), `iters` times; lane 0 of each wave records
// the shader-clock cycles (s_memtime) of its loop.  The loaded values are consumed by an empty asm
// statement (no VALU work beside the reads) and the offsets pass through one each iteration, so
// the reads are neither hoisted nor narrowed.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int PROBE_WAVES = 16;
constexpr int PROBE_READS = 8;
constexpr int TILE_SLOTS16 = 4096;  // 64 KiB of 16-byte slots

template <int BYTES>
__global__ void __launch_bounds__(PROBE_WAVES * 64) lds_probe_kernel(const uint32_t* __restrict__ offs, int iters,
                                                                     unsigned long long* __restrict__ cycles) {
  __shared__ float4 tile[TILE_SLOTS16];
  for (int i = threadIdx.x; i < TILE_SLOTS16; i += PROBE_WAVES * 64)
    tile[i] = make_float4((float)i, (float)(i + 1), (float)(i + 2), (float)(i + 3));
  __syncthreads();
  const int lane = threadIdx.x & 63;
  uint32_t a[PROBE_READS];
#pragma unroll
  for (int r = 0; r < PROBE_READS; ++r) a[r] = offs[r * 64 + lane] & (TILE_SLOTS16 * 16 - BYTES);  // in the tile, aligned
  const char* base = reinterpret_cast<const char*>(tile);
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < PROBE_READS; ++r) asm volatile("" : "+v"(a[r]));
    if constexpr (BYTES == 16) {
      float4 v[PROBE_READS];
#pragma unroll
      for (int r = 0; r < PROBE_READS; ++r) v[r] = *reinterpret_cast<const float4*>(base + a[r]);
#pragma unroll
      for (int r = 0; r < PROBE_READS; ++r) asm volatile("" ::"v"(v[r].x), "v"(v[r].y), "v"(v[r].z), "v"(v[r].w));
    } else {
      float2 v[PROBE_READS];
#pragma unroll
      for (int r = 0; r < PROBE_READS; ++r) v[r] = *reinterpret_cast<const float2*>(base + a[r]);
#pragma unroll
      for (int r = 0; r < PROBE_READS; ++r) asm volatile("" ::"v"(v[r].x), "v"(v[r].y));
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  if (lane == 0) cycles[(long long)blockIdx.x * PROBE_WAVES + (threadIdx.x >> 6)] = t1 - t0;
}

}  // namespace

// offs: 8 x 64 byte offsets into the tile (device memory); cycles: blocks x 16 entries (device
// memory).  Returns 0, or -1 for an unsupported slot size or launch shape.
extern "C" int gl_lds_probe(int bytes, const void* offs, int iters, void* cycles, int blocks, void* stream) {
  if ((bytes != 8 && bytes != 16) || iters < 1 || blocks < 1 || !offs || !cycles) return -1;
  hipStream_t s = (hipStream_t)stream;
  if (bytes == 16)
    hipLaunchKernelGGL(lds_probe_kernel<16>, dim3((unsigned)blocks), dim3(PROBE_WAVES * 64), 0, s,
                       (const uint32_t*)offs, iters, (unsigned long long*)cycles);
  else
    hipLaunchKernelGGL(lds_probe_kernel<8>, dim3((unsigned)blocks), dim3(PROBE_WAVES * 64), 0, s,
                       (const uint32_t*)offs, iters, (unsigned long long*)cycles);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
