// gfx950 LDS helpers shared by the direct-to-LDS kernels (the f32/f16 GEMMs, f16 attention):
// global->LDS loads, explicit vector-memory waits, and transposed 16-bit LDS reads.
#pragma once

#include "device.h"

namespace msx::hk {
namespace {
#define MSX_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))
// 16 bytes a lane from global memory into LDS at dst + 16 lane (the host pass sees an empty body).
__device__ __forceinline__ void load_lds16(const void* src, void* dst) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(src, MSX_LDS_PTR(dst), 16, 0, 0);
#endif
}
// Waits until at most n vector memory operations of this wave are outstanding (expcnt and lgkmcnt
// unconstrained).
__device__ __forceinline__ void wait_vm(int n) {
  switch (n) {
#define MSX_W(N) case N: __builtin_amdgcn_s_waitcnt(((N) & 0xF) | (((N) >> 4) << 14) | (7 << 4) | (0xF << 8)); break;
    MSX_W(0) MSX_W(1) MSX_W(2) MSX_W(3) MSX_W(4) MSX_W(5) MSX_W(6) MSX_W(7) MSX_W(8) MSX_W(9) MSX_W(10)
    MSX_W(11) MSX_W(12) MSX_W(13) MSX_W(14) MSX_W(15) MSX_W(16) MSX_W(17) MSX_W(18) MSX_W(19) MSX_W(20)
    MSX_W(21) MSX_W(22) MSX_W(23) MSX_W(24)
#undef MSX_W
    default: __builtin_amdgcn_s_waitcnt((7 << 4) | (0xF << 8)); break;
  }
}

typedef short v4s16 __attribute__((ext_vector_type(4)));
typedef _Float16 v4h16 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t lds_at(const _Float16* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}
// Eight transposed reads (ds_read_b64_tr_b16) and the wait for them, as one block of inline
// assembly: through the builtin the compiler waits for every global->LDS load in flight (vmcnt(0),
// the prefetches too) before each transposed read, and separate asm reads would let it use their
// registers before the data arrives. In each 16-lane group, source lane l reads 8 bytes (4
// halves) at at[u]; destination lane l's half j is source lane (4 j + l / 4)'s half l mod 4.
__device__ __forceinline__ void tr_read16x8(const uint32_t (&at)[8], v4s16 (&r)[8]) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8\n"
      "ds_read_b64_tr_b16 %1, %9\n"
      "ds_read_b64_tr_b16 %2, %10\n"
      "ds_read_b64_tr_b16 %3, %11\n"
      "ds_read_b64_tr_b16 %4, %12\n"
      "ds_read_b64_tr_b16 %5, %13\n"
      "ds_read_b64_tr_b16 %6, %14\n"
      "ds_read_b64_tr_b16 %7, %15\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
      : "v"(at[0]), "v"(at[1]), "v"(at[2]), "v"(at[3]), "v"(at[4]), "v"(at[5]), "v"(at[6]), "v"(at[7])
      : "memory");
#endif
}
// The same eight reads without the wait: r is not to be read before lds_wait8(r), which waits
// for them and, taking r as its operands, keeps every use of r after it.
__device__ __forceinline__ void tr_issue16x8(const uint32_t (&at)[8], v4s16 (&r)[8]) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8\n"
      "ds_read_b64_tr_b16 %1, %9\n"
      "ds_read_b64_tr_b16 %2, %10\n"
      "ds_read_b64_tr_b16 %3, %11\n"
      "ds_read_b64_tr_b16 %4, %12\n"
      "ds_read_b64_tr_b16 %5, %13\n"
      "ds_read_b64_tr_b16 %6, %14\n"
      "ds_read_b64_tr_b16 %7, %15"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
      : "v"(at[0]), "v"(at[1]), "v"(at[2]), "v"(at[3]), "v"(at[4]), "v"(at[5]), "v"(at[6]), "v"(at[7])
      : "memory");
#endif
}
__device__ __forceinline__ void lds_wait8(v4s16 (&r)[8]) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7])
               :
               : "memory");
#endif
}

// Four 16-byte LDS reads and the wait for them, in inline assembly for the reason above: LDS
// the global->LDS loads do not write, read without waiting for those loads.
__device__ __forceinline__ void lds_read4x16(const uint32_t (&at)[4], float4 (&r)[4]) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef float v4f_ __attribute__((ext_vector_type(4)));
  v4f_ x0, x1, x2, x3;
  asm volatile(
      "ds_read_b128 %0, %4\n"
      "ds_read_b128 %1, %5\n"
      "ds_read_b128 %2, %6\n"
      "ds_read_b128 %3, %7\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3)
      : "v"(at[0]), "v"(at[1]), "v"(at[2]), "v"(at[3])
      : "memory");
  r[0] = make_float4(x0[0], x0[1], x0[2], x0[3]);
  r[1] = make_float4(x1[0], x1[1], x1[2], x1[3]);
  r[2] = make_float4(x2[0], x2[1], x2[2], x2[3]);
  r[3] = make_float4(x3[0], x3[1], x3[2], x3[3]);
#endif
}
__device__ __forceinline__ uint32_t lds_at(const float* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}
}  // namespace
}  // namespace msx::hk
