// Device pieces shared by the two GEMM sources (gemm.hip, gemm_lds.hip): the output epilogue and
// the tile order, and the large-shape kernel's launcher.
#pragma once
#include "kernels.h"
#include "device.h"

namespace msx::hk {

// The output epilogue of element (row, col) of a product v: + bias[col], then the activation
// (GELU or ReLU, the pre-activation value also stored to pre_out when asked; or their gradient
// with respect to the pre-activation pre_in[row, col], v the incoming gradient), then addend[row,
// col] + v, then the dropout gradient (kept or zeroed by the dropout kernel's rule at the
// element's index). Every step rounds as the separate kernel would (the same operation order).
// With pre16 the pre-activation is kept as f16 instead (written rounded, read widened).
__device__ __forceinline__ float epi_drop(const GemmEpi& e, float v, int64_t at) {
  const uint32_t w = philox_w0(uint32_t(at), 4u, uint32_t(e.drop_token[0]), uint32_t(e.drop_token[1]),
                               uint32_t(e.drop_seed), uint32_t(e.drop_seed >> 32));
  return uint64_t(w) >= e.drop_threshold ? v * e.drop_scale : 0.0f;
}
__device__ __forceinline__ float gemm_epilogue(const GemmEpi& e, float v, int64_t row, int64_t col, int64_t ldc) {
  if (e.bias) v = v + e.bias[col];
  const int64_t at = row * ldc + col;
  switch (e.act) {
    case EPI_GELU:
      if (e.pre16) e.pre16[at] = _Float16(v);
      else if (e.pre_out) e.pre_out[at] = v;
      v = d_gelu(v);
      break;
    case EPI_RELU:
      if (e.pre16) e.pre16[at] = _Float16(v);
      else if (e.pre_out) e.pre_out[at] = v;
      v = v > 0.0f ? v : 0.0f;
      break;
    case EPI_GELU_GRAD: v = d_gelu_grad(e.pre16 ? float(e.pre16[at]) : e.pre_in[at], v); break;
    case EPI_RELU_GRAD: v = (e.pre16 ? float(e.pre16[at]) : e.pre_in[at]) > 0.0f ? v : 0.0f; break;
    default: break;
  }
  if (e.addend) v = e.addend[at] + v;
  if (e.drop_token) v = epi_drop(e, v, at);
  return v;
}
// The same on four consecutive columns (col a multiple of 4, 16-byte aligned rows).
__device__ __forceinline__ float4 gemm_epilogue4(const GemmEpi& e, float4 v, int64_t row, int64_t col, int64_t ldc) {
  if (e.bias) {
    const float4 b = *reinterpret_cast<const float4*>(e.bias + col);
    v = make_float4(v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w);
  }
  const int64_t at = row * ldc + col;
  typedef _Float16 h4_ __attribute__((ext_vector_type(4)));
  auto put_pre = [&]() {
    if (e.pre16) *reinterpret_cast<h4_*>(e.pre16 + at) = h4_{_Float16(v.x), _Float16(v.y), _Float16(v.z), _Float16(v.w)};
    else if (e.pre_out) *reinterpret_cast<float4*>(e.pre_out + at) = v;
  };
  auto get_pre = [&]() {
    if (!e.pre16) return *reinterpret_cast<const float4*>(e.pre_in + at);
    const h4_ h = *reinterpret_cast<const h4_*>(e.pre16 + at);
    return make_float4(float(h[0]), float(h[1]), float(h[2]), float(h[3]));
  };
  switch (e.act) {
    case EPI_GELU:
      put_pre();
      v = make_float4(d_gelu(v.x), d_gelu(v.y), d_gelu(v.z), d_gelu(v.w));
      break;
    case EPI_RELU:
      put_pre();
      v = make_float4(v.x > 0.0f ? v.x : 0.0f, v.y > 0.0f ? v.y : 0.0f, v.z > 0.0f ? v.z : 0.0f, v.w > 0.0f ? v.w : 0.0f);
      break;
    case EPI_GELU_GRAD: {
      const float4 p = get_pre();
      v = make_float4(d_gelu_grad(p.x, v.x), d_gelu_grad(p.y, v.y), d_gelu_grad(p.z, v.z), d_gelu_grad(p.w, v.w));
      break;
    }
    case EPI_RELU_GRAD: {
      const float4 p = get_pre();
      v = make_float4(p.x > 0.0f ? v.x : 0.0f, p.y > 0.0f ? v.y : 0.0f, p.z > 0.0f ? v.z : 0.0f, p.w > 0.0f ? v.w : 0.0f);
      break;
    }
    default: break;
  }
  if (e.addend) {
    const float4 a = *reinterpret_cast<const float4*>(e.addend + at);
    v = make_float4(a.x + v.x, a.y + v.y, a.z + v.z, a.w + v.w);
  }
  if (e.drop_token)
    v = make_float4(epi_drop(e, v.x, at), epi_drop(e, v.y, at + 1), epi_drop(e, v.z, at + 2), epi_drop(e, v.w, at + 3));
  return v;
}

// The order a GEMM's tiles are handed to blocks: mt x nt tiles a split slice, `tiles` in all (of
// one problem of the group), M tiles adjacent when m_fastest.
struct GemmOrder {
  uint32_t mt, nt, tiles;
  bool m_fastest;
};

// Launches the direct-to-LDS kernel for one f32 problem (no K segments, no cross-entropy operand)
// with the caller's split-K slices (`split` slices of `chunk` K, partials in ptrs.ws[0]) when its
// shape and layout suit it; returns false, launching nothing, otherwise.
bool gemm_lds(hipStream_t s, const GemmArgs& g, const GemmPtrs& ptrs, int split, int64_t chunk);
// The same for a mixed-precision group whose operands all have f16 copies (GemmArgs::a16, b16):
// the f16 kernel reads them straight into LDS; it writes the f32 output (or split-K partials) and
// the f16 output copies asked for.
bool gemm_lds16(hipStream_t s, const GemmArgs* list, int count, const GemmPtrs& ptrs, int split, int64_t chunk);
// Whether k_gemm_lds16 takes a problem of this shape and layout with split-K slices of `chunk`
// (its f16 operand copies present and 16-byte aligned aside).
bool lds16_layout(const GemmArgs& g, int64_t chunk);

}  // namespace msx::hk
