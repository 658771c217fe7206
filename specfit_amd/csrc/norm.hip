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
// otherwise one element per lane step.  x and out may be the same rows (an
// in-place call), so neither is declared __restrict__.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const uint16_t* x,
                                                            int64_t row_stride, int rows, int dim,
                                                            const uint16_t* __restrict__ weight,
                                                            float eps, uint16_t* out,
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

// ------------------------------------------------------------------ K7 ----
// Query/key RMSNorm and rotary embedding of one attention layer, fused.
// Restates, for head_dim 128 and batch 1,
//   q = q_norm(q_proj(h).view(T, Hq, D)), k = k_norm(k_proj(h).view(T, Hk, D))
//   (Qwen3MoeAttention.forward, tf:162-163) and apply_rotary_pos_emb
//   (tf:58-81) with rotate_half (tf:51-55):
//   x_embed[d] = bf16(bf16(x[d] * cos[t, d]) + bf16(rot(x)[d] * sin[t, d])),
//   rot(x)[d] = -x[d + 64] for d < 64, x[d - 64] otherwise,
// where x is the normed row.  Each eager operation rounds to bf16, so the
// fused form reproduces them exactly; the norm is K6's (same lane layout and
// summation order, so the same bits).  The eager form is twelve kernels per
// layer (two norms, then per tensor a negation, a concatenation, two
// products and a sum).
//
// A row (one token's head) is 16 lanes x 8 elements; a wavefront takes four
// rows, so the norm's sum is the 16-lane butterfly K6 applies to a
// 128-element row, and the rotation partner of lane j's elements (d +- 64)
// sits in lane j ^ 8 of the same 16-lane row (one DPP row rotation).
// Outputs are written head-major: out[h][t][d].
namespace {

constexpr int kRopeDim = 128;

__device__ __forceinline__ float row16_sum(float x) {
  x += sf_dpp<0xB1>(x);   // lane ^ 1
  x += sf_dpp<0x4E>(x);   // lane ^ 2
  x += sf_dpp<0x141>(x);  // row_half_mirror
  x += sf_dpp<0x140>(x);  // row_mirror
  return x;
}

__global__ __launch_bounds__(kThreads) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ q, int64_t q_tok, const uint16_t* __restrict__ k, int64_t k_tok,
    int tokens, int q_heads,
    int kv_heads, const uint16_t* __restrict__ wq, const uint16_t* __restrict__ wk, float eps,
    const uint16_t* __restrict__ cos, const uint16_t* __restrict__ sin,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out) {
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int j = lane & 15;
  const int q_rows = tokens * q_heads;
  const int rows = q_rows + tokens * kv_heads;
  const int row = (blockIdx.x * kThreads + threadIdx.x) / 16;
  // Rows past the end repeat the last row's loads (no store): the DPP moves
  // below need every lane of the 16-lane row active.
  const bool live = row < rows;
  const int r = live ? row : rows - 1;
  const bool is_q = r < q_rows;
  const int rr = is_q ? r : r - q_rows;
  const int heads = is_q ? q_heads : kv_heads;
  const int t = rr / heads;
  const int h = rr - t * heads;
  const uint16_t* src = (is_q ? q : k) + static_cast<int64_t>(t) * (is_q ? q_tok : k_tok) +
                        static_cast<int64_t>(h) * kRopeDim;
  const uint16_t* w = is_q ? wq : wk;
  float f[8], g[8], c[8], s[8];
  unpack(ld16(src + 8 * j), f);
  unpack(ld16(w + 8 * j), g);
  unpack(ld16(cos + static_cast<int64_t>(t) * kRopeDim + 8 * j), c);
  unpack(ld16(sin + static_cast<int64_t>(t) * kRopeDim + 8 * j), s);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
  const float var = row16_sum(ss) * (1.0f / static_cast<float>(kRopeDim));
  const float rs = __builtin_amdgcn_rsqf(var + eps);
  float n[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) n[i] = sf_round_bf16(g[i] * sf_round_bf16(f[i] * rs));
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    float e[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float partner = sf_dpp<0x128>(n[i + u]);  // row_ror 8: lane j ^ 8
      const float rot = j < 8 ? -partner : partner;
      e[u] = sf_round_bf16(sf_round_bf16(n[i + u] * c[i + u]) + sf_round_bf16(rot * s[i + u]));
    }
    o[i / 2] = static_cast<uint32_t>(sf_f32_to_bf16(e[0])) |
               (static_cast<uint32_t>(sf_f32_to_bf16(e[1])) << 16);
  }
  if (live) {
    uint16_t* dst = (is_q ? q_out : k_out) +
                    (static_cast<int64_t>(h) * tokens + t) * kRopeDim + 8 * j;
    *reinterpret_cast<uint4*>(dst) = uint4{o[0], o[1], o[2], o[3]};
  }
}

}  // namespace

extern "C" int sf_qk_norm_rope(const void* q, int64_t q_stride_token, const void* k,
                               int64_t k_stride_token, int tokens, int q_heads,
                               int kv_heads, int head_dim, const void* q_weight,
                               const void* k_weight, float eps, const void* cos, const void* sin,
                               void* q_out, void* k_out, sf_stream_t stream) {
  if (tokens < 0 || q_heads < 1 || kv_heads < 1 || !(eps >= 0.f)) return SF_ERR_INVALID_ARGUMENT;
  if (head_dim != kRopeDim) return SF_ERR_UNSUPPORTED_SHAPE;
  if (q_stride_token < static_cast<int64_t>(q_heads) * kRopeDim ||
      k_stride_token < static_cast<int64_t>(kv_heads) * kRopeDim || q_stride_token % 8 ||
      k_stride_token % 8)
    return SF_ERR_INVALID_ARGUMENT;
  if (tokens == 0) return SF_OK;
  const void* ptrs[] = {q, k, q_weight, k_weight, cos, sin, q_out, k_out};
  for (const void* p : ptrs)
    if (!p || !aligned16(p)) return SF_ERR_INVALID_ARGUMENT;
  const long long rows = static_cast<long long>(tokens) * (q_heads + kv_heads);
  if (rows > 0x7fffffffLL / 16) return SF_ERR_UNSUPPORTED_SHAPE;
  const unsigned blocks = static_cast<unsigned>((rows * 16 + kThreads - 1) / kThreads);
  qk_norm_rope_kernel<<<dim3(blocks), dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(q), q_stride_token, static_cast<const uint16_t*>(k),
      k_stride_token, tokens, q_heads, kv_heads,
      static_cast<const uint16_t*>(q_weight), static_cast<const uint16_t*>(k_weight), eps,
      static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin),
      static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out));
  SF_LAUNCH_CHECK();
  return SF_OK;
}
