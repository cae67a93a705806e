// Device helpers shared by the kernel sources of the training step (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace msx::hk {

// The kernels a host thread dispatches are noted while a log is attached (profiling: which HIP
// kernels one planned launch ran).
void note_kernel(const char* expr);
#define MSX_LAUNCH(KERNEL, ...)                 \
  do {                                          \
    ::msx::hk::note_kernel(#KERNEL);            \
    hipLaunchKernelGGL(KERNEL, __VA_ARGS__);    \
  } while (0)

namespace {
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

[[noreturn]] void bad(const std::string& what) { throw std::runtime_error("kernel launch refused: " + what); }

inline unsigned blocks_for(int64_t n, int per) { return unsigned((n + per - 1) / per); }

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// The GELU of interpreter.rs:1539-1587 in device arithmetic: the nearest f32 constants, the same
// operation order, the device expf.
__device__ __forceinline__ float d_gelu_twice_inner(float x) {
  const float scale = 0.797884560802865f, cubic = 0.044715f;
  return 2.0f * scale * (x + cubic * x * x * x);
}
__device__ __forceinline__ float d_logistic(float v) { return 1.0f / (1.0f + expf(0.0f - v)); }
__device__ __forceinline__ float d_gelu(float x) { return x * d_logistic(d_gelu_twice_inner(x)); }
__device__ __forceinline__ float d_gelu_grad(float x, float g) {
  const float scale = 0.797884560802865f, cubic = 0.044715f;
  float v = d_gelu_twice_inner(x);
  float s = d_logistic(v), r = d_logistic(0.0f - v);
  float slope = scale * (1.0f + 3.0f * cubic * x * x);
  return (s + 2.0f * (s * x) * r * slope) * g;
}

// Philox4x32-10 word 0 (train/init.rs:91-109), on the device for the dropout masks.
__device__ __forceinline__ uint32_t philox_w0(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                              uint32_t k1) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int round = 0; round < 10; ++round) {
    if (round > 0) { k0 += W0; k1 += W1; }
    // 32 x 32 -> 64-bit products: one v_mad_u64_u32 gives both halves (a mul_hi / mul_lo pair costs two).
    const uint64_t p0 = uint64_t(M0) * c0, p1 = uint64_t(M1) * c2;
    const uint32_t n0 = uint32_t(p1 >> 32) ^ c1 ^ k0, n2 = uint32_t(p0 >> 32) ^ c3 ^ k1;
    c0 = n0; c1 = uint32_t(p1); c2 = n2; c3 = uint32_t(p0);
  }
  return c0;
}
// All four words of the same block.
__device__ __forceinline__ uint4 philox_block4(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                               uint32_t k1) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int round = 0; round < 10; ++round) {
    if (round > 0) { k0 += W0; k1 += W1; }
    // 32 x 32 -> 64-bit products: one v_mad_u64_u32 gives both halves (a mul_hi / mul_lo pair costs two).
    const uint64_t p0 = uint64_t(M0) * c0, p1 = uint64_t(M1) * c2;
    const uint32_t n0 = uint32_t(p1 >> 32) ^ c1 ^ k0, n2 = uint32_t(p0 >> 32) ^ c3 ^ k1;
    c0 = n0; c1 = uint32_t(p1); c2 = n2; c3 = uint32_t(p0);
  }
  return make_uint4(c0, c1, c2, c3);
}
}  // namespace

}  // namespace msx::hk
