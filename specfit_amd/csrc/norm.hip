// K6: RMSNorm of the verification forward's dense layers on gfx950.
// Restates Qwen3MoeRMSNorm.forward (tf:294-299; "tf:" is
// transformers/models/qwen3_moe/modeling_qwen3_moe.py):
//   v   = mean(float(x)^2)            over the last dimension, fp32
//   y   = bf16(float(x) * rsqrt(v + eps))
//   out = bf16(float(weight) * float(y))
// with the same two bf16 rounding points.  Every decoder layer runs four of
// them (input, post-attention, and the per-head query and key norms), and
// the eager form is seven or eight elementwise/reduction kernels each, ~4.5
// us apiece on MI355X however small the tensor: one kernel per norm instead.
//
// One wavefront per row: lane l takes the 8-element chunks l, l + 64, ...,
// sums their squares in chunk order, and the wavefront adds the 64 partial
// sums by the xor butterfly of sf_wave_sum.  The second pass re-reads the row
// (an L1/L2 hit) and writes the output.  The summation order differs from
// torch's reduction, so results match the eager module within a last-place
// rounding of the variance (tests bound the difference).
#include "sf_common.h"

namespace {

constexpr int kRowsPerBlock = 4;
constexpr int kThreads = kRowsPerBlock * SF_WAVE;

typedef unsigned int sf_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld16(const uint16_t* p) {
  const sf_u32x4 v = *(const __attribute__((address_space(1))) sf_u32x4*)(p);
  return __builtin_bit_cast(uint4, v);
}

__device__ __forceinline__ void unpack(uint4 v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// VEC: rows are 16-byte aligned and dim % 8 == 0 (8-element chunks);
// otherwise one element per lane step.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const uint16_t* __restrict__ x,
                                                            int64_t row_stride, int rows, int dim,
                                                            const uint16_t* __restrict__ weight,
                                                            float eps, uint16_t* __restrict__ out,
                                                            int64_t out_stride) {
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int row = blockIdx.x * kRowsPerBlock + threadIdx.x / SF_WAVE;
  if (row >= rows) return;  // wave-uniform
  const uint16_t* xr = x + static_cast<int64_t>(row) * row_stride;
  uint16_t* orow = out + static_cast<int64_t>(row) * out_stride;
  float ss = 0.f;
  if (VEC) {
    const int chunks = dim / 8;
    for (int c = lane; c < chunks; c += SF_WAVE) {
      float f[8];
      unpack(ld16(xr + 8 * c), f);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
    }
  } else {
    for (int k = lane; k < dim; k += SF_WAVE) {
      const float f = sf_bf16_to_f32(xr[k]);
      ss = __builtin_fmaf(f, f, ss);
    }
  }
  // mean as torch's reduction projects it: the sum times 1/dim.
  const float var = sf_wave_sum(ss) * (1.0f / static_cast<float>(dim));
  const float r = __builtin_amdgcn_rsqf(var + eps);
  if (VEC) {
    const int chunks = dim / 8;
    for (int c = lane; c < chunks; c += SF_WAVE) {
      float f[8], g[8];
      unpack(ld16(xr + 8 * c), f);
      unpack(ld16(weight + 8 * c), g);
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float y0 = sf_round_bf16(f[2 * i] * r);
        const float y1 = sf_round_bf16(f[2 * i + 1] * r);
        o[i] = static_cast<uint32_t>(sf_f32_to_bf16(g[2 * i] * y0)) |
               (static_cast<uint32_t>(sf_f32_to_bf16(g[2 * i + 1] * y1)) << 16);
      }
      *reinterpret_cast<uint4*>(orow + 8 * c) = uint4{o[0], o[1], o[2], o[3]};
    }
  } else {
    for (int k = lane; k < dim; k += SF_WAVE) {
      const float y = sf_round_bf16(sf_bf16_to_f32(xr[k]) * r);
      orow[k] = sf_f32_to_bf16(sf_bf16_to_f32(weight[k]) * y);
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int sf_rms_norm(const void* x, int64_t row_stride, int rows, int dim,
                           const void* weight, float eps, void* out, int64_t out_stride,
                           sf_stream_t stream) {
  if (rows < 0 || dim < 1 || row_stride < dim || out_stride < dim || !(eps >= 0.f))
    return SF_ERR_INVALID_ARGUMENT;
  if (rows == 0) return SF_OK;
  if (!x || !weight || !out) return SF_ERR_INVALID_ARGUMENT;
  const bool vec = dim % 8 == 0 && row_stride % 8 == 0 && out_stride % 8 == 0 && aligned16(x) &&
                   aligned16(weight) && aligned16(out);
  const unsigned blocks = static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint16_t*>(weight);
  auto* op = static_cast<uint16_t*>(out);
  if (vec)
    rms_norm_kernel<true><<<dim3(blocks), dim3(kThreads), 0, s>>>(xp, row_stride, rows, dim, wp,
                                                                  eps, op, out_stride);
  else
    rms_norm_kernel<false><<<dim3(blocks), dim3(kThreads), 0, s>>>(xp, row_stride, rows, dim, wp,
                                                                   eps, op, out_stride);
  SF_LAUNCH_CHECK();
  return SF_OK;
}
