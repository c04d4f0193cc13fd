// Fused AdamW over fp32 parameters: one streaming pass reads p, g, m, v and writes p, m, v and
// g = 0 (32 bytes per element with fp32 moments, 24 with bf16 moments).
// Reference: _adamw_kernel, sparse_pooling/optim.py:26-64 (HAS_MASTER = STOCH = False).  The
// update is evaluated unfused in the reference's operation order; every element is read and
// written by the same thread, so the in-place race fixed at optim.py:43-50 cannot occur.
#include "gl_common.h"
#include "gl_internal.h"

namespace gl {

struct AdamK {
  float lr, b1, b2, eps, wd, bc1, bc2;
};

__device__ __forceinline__ float bf16_bits_to_f32(unsigned short u) { return __uint_as_float((unsigned)u << 16); }
__device__ __forceinline__ unsigned short f32_to_bf16_rne(float f) {
  unsigned u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) return (unsigned short)((u | ((u & 0x007fffffu) ? 0x00400000u : 0u)) >> 16);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (unsigned short)(u >> 16);
}

__device__ __forceinline__ void adam_elem(const AdamK& c, float& p, float g, float& m, float& v) {
#pragma clang fp contract(off)
  m = c.b1 * m + (1.0f - c.b1) * g;
  v = c.b2 * v + (1.0f - c.b2) * g * g;
  const float upd = (m / c.bc1) / (__builtin_sqrtf(v / c.bc2) + c.eps);
  p = p * (1.0f - c.lr * c.wd) - c.lr * upd;
}

template <bool BF16M>
__global__ void __launch_bounds__(256) adam_kernel(float* __restrict__ P, float* __restrict__ Gr, void* __restrict__ M,
                                                   void* __restrict__ V, long long n, AdamK c) {
  const long long n4 = n >> 2;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    float4 p = reinterpret_cast<float4*>(P)[i];
    const float4 g = reinterpret_cast<const float4*>(Gr)[i];
    float4 m, v;
    if constexpr (BF16M) {
      const ushort4 mb = reinterpret_cast<const ushort4*>(M)[i];
      const ushort4 vb = reinterpret_cast<const ushort4*>(V)[i];
      m = make_float4(bf16_bits_to_f32(mb.x), bf16_bits_to_f32(mb.y), bf16_bits_to_f32(mb.z), bf16_bits_to_f32(mb.w));
      v = make_float4(bf16_bits_to_f32(vb.x), bf16_bits_to_f32(vb.y), bf16_bits_to_f32(vb.z), bf16_bits_to_f32(vb.w));
    } else {
      m = reinterpret_cast<const float4*>(M)[i];
      v = reinterpret_cast<const float4*>(V)[i];
    }
    adam_elem(c, p.x, g.x, m.x, v.x);
    adam_elem(c, p.y, g.y, m.y, v.y);
    adam_elem(c, p.z, g.z, m.z, v.z);
    adam_elem(c, p.w, g.w, m.w, v.w);
    if constexpr (BF16M) {
      reinterpret_cast<ushort4*>(M)[i] = make_ushort4(f32_to_bf16_rne(m.x), f32_to_bf16_rne(m.y), f32_to_bf16_rne(m.z),
                                                      f32_to_bf16_rne(m.w));
      reinterpret_cast<ushort4*>(V)[i] = make_ushort4(f32_to_bf16_rne(v.x), f32_to_bf16_rne(v.y), f32_to_bf16_rne(v.z),
                                                      f32_to_bf16_rne(v.w));
    } else {
      reinterpret_cast<float4*>(M)[i] = m;
      reinterpret_cast<float4*>(V)[i] = v;
    }
    reinterpret_cast<float4*>(Gr)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    reinterpret_cast<float4*>(P)[i] = p;
  }
  // tail (n % 4 elements), handled by the first threads of block 0
  const long long t = (n4 << 2) + threadIdx.x;
  if (blockIdx.x == 0 && t < n) {
    float p = P[t], g = Gr[t], m, v;
    if constexpr (BF16M) {
      m = bf16_bits_to_f32(reinterpret_cast<unsigned short*>(M)[t]);
      v = bf16_bits_to_f32(reinterpret_cast<unsigned short*>(V)[t]);
    } else {
      m = reinterpret_cast<float*>(M)[t];
      v = reinterpret_cast<float*>(V)[t];
    }
    adam_elem(c, p, g, m, v);
    if constexpr (BF16M) {
      reinterpret_cast<unsigned short*>(M)[t] = f32_to_bf16_rne(m);
      reinterpret_cast<unsigned short*>(V)[t] = f32_to_bf16_rne(v);
    } else {
      reinterpret_cast<float*>(M)[t] = m;
      reinterpret_cast<float*>(V)[t] = v;
    }
    Gr[t] = 0.f;
    P[t] = p;
  }
}

}  // namespace gl

using namespace gl;

extern "C" int gl_adam(const GlAdamArgs* a, void* stream) {
  if (!a || a->n < 0) return GL_ERR_ARG;
  if (a->n == 0) return 0;
  if (!a->p || !a->g || !a->m || !a->v) return GL_ERR_ARG;
  if (a->moments_dtype != GL_DTYPE_F32 && a->moments_dtype != GL_DTYPE_BF16) return GL_ERR_UNSUPPORTED;
  // vector path needs 16-byte (8-byte for bf16 moments) alignment
  const uintptr_t al = (uintptr_t)a->p | (uintptr_t)a->g;
  const uintptr_t alm = (uintptr_t)a->m | (uintptr_t)a->v;
  if ((al & 15) || (alm & (a->moments_dtype == GL_DTYPE_F32 ? 15 : 7))) return GL_ERR_ARG;
  AdamK c{a->lr, a->beta1, a->beta2, a->eps, a->weight_decay, a->bc1, a->bc2};
  hipStream_t s = (hipStream_t)stream;
  long long n4 = a->n >> 2;
  long long blocks = (n4 + 255) / 256;
  if (blocks > 256 * 16) blocks = 256 * 16;
  if (blocks < 1) blocks = 1;
  if (a->moments_dtype == GL_DTYPE_F32)
    GL_LAUNCH(GL_KERNEL_ADAM, adam_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, a->p, a->g, a->m, a->v, a->n, c);
  else
    GL_LAUNCH(GL_KERNEL_ADAM, adam_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, a->p, a->g, a->m, a->v, a->n, c);
  GL_CHECK_LAUNCH();
  return 0;
}
