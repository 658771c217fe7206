// K1: fused router -- bf16 logits, fp32 softmax, top-k with wavefront-shuffle
// argmax, optional renormalisation.  Restates Qwen3MoeTopKRouter.forward
// (transformers qwen3_moe modeling file, tf:258-267) for gfx950.
//
// Arithmetic contract (the CPU oracle evaluates exactly this):
//  * logit[t,e]: lane l of a 64-wide wavefront owns the 8-element chunks
//    c = l, l+64, l+128, ... of the hidden dimension and accumulates
//    hidden[k]*W[e,k] for its k in ascending order into an fp32 partial that
//    starts at +0 (bf16*bf16 products are exact in fp32, so fused and unfused
//    accumulation agree).  The 64 partials are combined by an xor butterfly
//    with distances 32,16,8,4,2,1 (v[l] += v[l^d]); the result is rounded to
//    bf16 (nearest even).
//  * softmax: m = max logit; x_e = exp(logit_e - m) with sf_exp_nonpos; lane l
//    owns experts l, l+64, l+128, l+192 and sums its x_e in that order from
//    +0, then the same butterfly combines lanes; p_e = x_e / sum (IEEE
//    division).
//  * top-k: k rounds of argmax over unselected experts with key
//    (p descending, expert id ascending).
//  * weights: v_j / (((v_0 + v_1) + v_2) + ...) when renormalising, else v_j,
//    rounded to bf16.
#include "sf_common.h"

namespace {

constexpr int kRouterThreads = 256;
constexpr int kRouterWaves = kRouterThreads / SF_WAVE;

__device__ __forceinline__ float wave_sum_butterfly(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, SF_WAVE);
  return v;
}

__device__ __forceinline__ float wave_max_butterfly(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, SF_WAVE));
  return v;
}

__device__ __forceinline__ float dot8_acc(uint4 hv, uint4 wv, float acc) {
  const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
  const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float h0 = __uint_as_float(hw[q] << 16);
    float w0 = __uint_as_float(ww[q] << 16);
    float h1 = __uint_as_float(hw[q] & 0xffff0000u);
    float w1 = __uint_as_float(ww[q] & 0xffff0000u);
    acc = __builtin_fmaf(h0, w0, acc);
    acc = __builtin_fmaf(h1, w1, acc);
  }
  return acc;
}

// Softmax + top-k + renorm over s_logit[0..E) by wavefront 0 of the block.
__device__ void softmax_topk_wave(const float* s_logit, int E, int K, int renorm,
                                  uint16_t* topw, int64_t* topi, float* s_val,
                                  int* s_id) {
  const int lane = threadIdx.x & (SF_WAVE - 1);
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < SF_MAX_EXPERTS / SF_WAVE; ++j) {
    int e = lane + SF_WAVE * j;
    if (e < E) m = fmaxf(m, s_logit[e]);
  }
  m = wave_max_butterfly(m);
  float x[SF_MAX_EXPERTS / SF_WAVE];
  float part = 0.0f;
#pragma unroll
  for (int j = 0; j < SF_MAX_EXPERTS / SF_WAVE; ++j) {
    int e = lane + SF_WAVE * j;
    if (e < E) {
      x[j] = sf_exp_nonpos(s_logit[e] - m);
      part += x[j];
    } else {
      x[j] = 0.0f;
    }
  }
  const float total = wave_sum_butterfly(part);
  float p[SF_MAX_EXPERTS / SF_WAVE];
  bool live[SF_MAX_EXPERTS / SF_WAVE];
#pragma unroll
  for (int j = 0; j < SF_MAX_EXPERTS / SF_WAVE; ++j) {
    int e = lane + SF_WAVE * j;
    live[j] = e < E;
    p[j] = live[j] ? x[j] / total : 0.0f;
  }
  for (int r = 0; r < K; ++r) {
    float bp = -1.0f;
    int be = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < SF_MAX_EXPERTS / SF_WAVE; ++j) {
      // ids grow with j inside a lane, so a strict comparison keeps the
      // lowest id among equal probabilities.
      if (live[j] && p[j] > bp) {
        bp = p[j];
        be = lane + SF_WAVE * j;
      }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      float op = __shfl_xor(bp, d, SF_WAVE);
      int oe = __shfl_xor(be, d, SF_WAVE);
      if (op > bp || (op == bp && oe < be)) {
        bp = op;
        be = oe;
      }
    }
    if ((be & (SF_WAVE - 1)) == lane) {
#pragma unroll
      for (int j = 0; j < SF_MAX_EXPERTS / SF_WAVE; ++j)
        if (be == lane + SF_WAVE * j) live[j] = false;
    }
    if (lane == 0) {
      s_val[r] = bp;
      s_id[r] = be;
    }
  }
  if (lane == 0) {
    float sum = 0.0f;
    for (int r = 0; r < K; ++r) sum += s_val[r];
    for (int r = 0; r < K; ++r) {
      float v = renorm ? s_val[r] / sum : s_val[r];
      topw[r] = sf_f32_to_bf16(v);
      topi[r] = static_cast<int64_t>(s_id[r]);
    }
  }
}

// Vector path: hidden_size % 8 == 0, 16-byte aligned rows, and at most
// NCH chunks of 8 elements per lane, so the token's hidden row stays in
// registers.  Sixteen wavefronts share the experts; each takes them four at
// a time with all router-weight loads of the four issued before any use, so
// the block is bound by one L2 round trip per group instead of one per
// expert.
constexpr int kRouterVecThreads = 1024;
constexpr int kRouterVecWaves = kRouterVecThreads / SF_WAVE;
// Experts per group: 16 uint4 router-weight registers per lane at most.
template <int NCH>
struct ExpertGroup {
  static constexpr int value = NCH <= 4 ? 4 : (NCH <= 8 ? 2 : 1);
};

template <int NCH>
__global__ __launch_bounds__(kRouterVecThreads) void router_topk_vec_kernel(
    const uint16_t* __restrict__ hidden, const uint16_t* __restrict__ wr, int H,
    int E, int K, int renorm, uint16_t* __restrict__ logits,
    uint16_t* __restrict__ topw, int64_t* __restrict__ topi) {
  constexpr int kExpertGroup = ExpertGroup<NCH>::value;
  __shared__ float s_logit[SF_MAX_EXPERTS];
  __shared__ float s_val[SF_MAX_TOPK];
  __shared__ int s_id[SF_MAX_TOPK];
  const int t = blockIdx.x;
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int nchunks = H / 8;
  const uint4* h4 = reinterpret_cast<const uint4*>(hidden + static_cast<size_t>(t) * H);
  uint4 hreg[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    int c = lane + SF_WAVE * i;
    hreg[i] = c < nchunks ? h4[c] : make_uint4(0, 0, 0, 0);
  }
  for (int e0 = wave * kExpertGroup; e0 < E; e0 += kRouterVecWaves * kExpertGroup) {
    uint4 wv[kExpertGroup][NCH];
#pragma unroll
    for (int g = 0; g < kExpertGroup; ++g) {
      const int e = min(e0 + g, E - 1);
      const uint4* w4 = reinterpret_cast<const uint4*>(wr + static_cast<size_t>(e) * H);
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        int c = lane + SF_WAVE * i;
        wv[g][i] = c < nchunks ? w4[c] : make_uint4(0, 0, 0, 0);
      }
    }
    float acc[kExpertGroup];
#pragma unroll
    for (int g = 0; g < kExpertGroup; ++g) {
      acc[g] = 0.0f;
#pragma unroll
      for (int i = 0; i < NCH; ++i)
        if (lane + SF_WAVE * i < nchunks) acc[g] = dot8_acc(hreg[i], wv[g][i], acc[g]);
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
#pragma unroll
      for (int g = 0; g < kExpertGroup; ++g) acc[g] += __shfl_xor(acc[g], d, SF_WAVE);
    }
    if (lane < kExpertGroup && e0 + lane < E) {
      float a = acc[0];
#pragma unroll
      for (int g = 1; g < kExpertGroup; ++g)
        if (lane == g) a = acc[g];
      const uint16_t b = sf_f32_to_bf16(a);
      logits[static_cast<size_t>(t) * E + e0 + lane] = b;
      s_logit[e0 + lane] = sf_bf16_to_f32(b);
    }
  }
  __syncthreads();
  if (wave == 0)
    softmax_topk_wave(s_logit, E, K, renorm, topw + static_cast<size_t>(t) * K,
                      topi + static_cast<size_t>(t) * K, s_val, s_id);
}

// Scalar path for any hidden_size / alignment: same summation order.
__global__ __launch_bounds__(kRouterThreads) void router_topk_scalar_kernel(
    const uint16_t* __restrict__ hidden, const uint16_t* __restrict__ wr, int H,
    int E, int K, int renorm, uint16_t* __restrict__ logits,
    uint16_t* __restrict__ topw, int64_t* __restrict__ topi) {
  __shared__ float s_logit[SF_MAX_EXPERTS];
  __shared__ float s_val[SF_MAX_TOPK];
  __shared__ int s_id[SF_MAX_TOPK];
  const int t = blockIdx.x;
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int nchunks = (H + 7) / 8;
  const uint16_t* h = hidden + static_cast<size_t>(t) * H;
  for (int e = wave; e < E; e += kRouterWaves) {
    const uint16_t* w = wr + static_cast<size_t>(e) * H;
    float acc = 0.0f;
    for (int c = lane; c < nchunks; c += SF_WAVE) {
      for (int j = 0; j < 8; ++j) {
        int k = c * 8 + j;
        if (k < H) acc = __builtin_fmaf(sf_bf16_to_f32(h[k]), sf_bf16_to_f32(w[k]), acc);
      }
    }
    acc = wave_sum_butterfly(acc);
    if (lane == 0) {
      uint16_t b = sf_f32_to_bf16(acc);
      logits[static_cast<size_t>(t) * E + e] = b;
      s_logit[e] = sf_bf16_to_f32(b);
    }
  }
  __syncthreads();
  if (wave == 0)
    softmax_topk_wave(s_logit, E, K, renorm, topw + static_cast<size_t>(t) * K,
                      topi + static_cast<size_t>(t) * K, s_val, s_id);
}

}  // namespace

extern "C" int sf_router_topk(const void* hidden, const void* router_weight,
                              int tokens, int hidden_size, int num_experts,
                              int top_k, int norm_topk_prob, void* logits,
                              void* topk_weights, int64_t* topk_index,
                              sf_stream_t stream) {
  if (tokens < 0 || hidden_size < 1 || num_experts < 1 ||
      num_experts > SF_MAX_EXPERTS || top_k < 1 || top_k > num_experts ||
      top_k > SF_MAX_TOPK)
    return SF_ERR_INVALID_ARGUMENT;
  if (tokens == 0) return SF_OK;
  if (!hidden || !router_weight || !logits || !topk_weights || !topk_index)
    return SF_ERR_INVALID_ARGUMENT;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint16_t* h = static_cast<const uint16_t*>(hidden);
  const uint16_t* w = static_cast<const uint16_t*>(router_weight);
  uint16_t* lg = static_cast<uint16_t*>(logits);
  uint16_t* tw = static_cast<uint16_t*>(topk_weights);
  const bool aligned = (reinterpret_cast<uintptr_t>(hidden) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(router_weight) % 16 == 0) &&
                       (hidden_size % 8 == 0);
  const int nchunks = (hidden_size + 7) / 8;
  const int per_lane = (nchunks + SF_WAVE - 1) / SF_WAVE;
  dim3 grid(tokens), block(kRouterThreads);
  if (aligned && per_lane <= 16) {
    block = dim3(kRouterVecThreads);
    if (per_lane <= 1)
      router_topk_vec_kernel<1><<<grid, block, 0, s>>>(h, w, hidden_size, num_experts, top_k, norm_topk_prob, lg, tw, topk_index);
    else if (per_lane <= 2)
      router_topk_vec_kernel<2><<<grid, block, 0, s>>>(h, w, hidden_size, num_experts, top_k, norm_topk_prob, lg, tw, topk_index);
    else if (per_lane <= 4)
      router_topk_vec_kernel<4><<<grid, block, 0, s>>>(h, w, hidden_size, num_experts, top_k, norm_topk_prob, lg, tw, topk_index);
    else if (per_lane <= 8)
      router_topk_vec_kernel<8><<<grid, block, 0, s>>>(h, w, hidden_size, num_experts, top_k, norm_topk_prob, lg, tw, topk_index);
    else
      router_topk_vec_kernel<16><<<grid, block, 0, s>>>(h, w, hidden_size, num_experts, top_k, norm_topk_prob, lg, tw, topk_index);
  } else {
    router_topk_scalar_kernel<<<grid, block, 0, s>>>(h, w, hidden_size, num_experts, top_k, norm_topk_prob, lg, tw, topk_index);
  }
  SF_LAUNCH_CHECK();
  return SF_OK;
}
