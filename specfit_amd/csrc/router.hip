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
//    with distances 1,2,4,8,16,32 (v[l] += v[l^d]); the result is rounded to
//    bf16 (nearest even).
//  * softmax: m = max logit; x_e = exp(logit_e - m) with sf_exp_nonpos; lane l
//    owns experts l, l+64, l+128, l+192 and sums its x_e in that order from
//    +0, then the same butterfly combines lanes; p_e = x_e / sum (IEEE
//    division).
//  * top-k: k rounds of argmax over unselected experts with key
//    (p descending, expert id ascending).
//  * weights: v_j / (((v_0 + v_1) + v_2) + ...) when renormalising, else v_j,
//    rounded to bf16.
// Wavefront reductions are DPP moves and lane reads (sf_wave_sum /
// sf_wave_max), which give exactly these butterfly sums.
#include "sf_common.h"

namespace {

constexpr int kRouterThreads = 256;
constexpr int kRouterWaves = kRouterThreads / SF_WAVE;

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

// Softmax + top-k + renorm over s_logit[0..E) by one wavefront.  Lane l
// reads only experts l, l+64, ... of s_logit.  Each top-k round takes the
// wave maximum of the unselected probabilities and the lowest expert id
// holding it (ballots per 64-expert slice, lowest lane first).  The rounds
// compare the probabilities' bit patterns as integers: p is in [0, 1] for
// finite logits, so integer order is float order and equal bits are equal
// values; -1 marks a slot past E or an expert already taken.  Lane r keeps
// round r's value and id, so the renormalisation divides in K lanes at once
// and the stores are contiguous.
template <int J>  // experts per lane: E <= 64 * J
__device__ void softmax_topk_wave(const float* s_logit, int E, int K, int renorm,
                                  uint16_t* topw, int64_t* topi) {
  const int lane = threadIdx.x & (SF_WAVE - 1);
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < J; ++j) {
    int e = lane + SF_WAVE * j;
    if (e < E) m = fmaxf(m, s_logit[e]);
  }
  m = sf_wave_max(m);
  float x[J];
  float part = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    int e = lane + SF_WAVE * j;
    if (e < E) {
      x[j] = sf_exp_nonpos(s_logit[e] - m);
      part += x[j];
    } else {
      x[j] = 0.0f;
    }
  }
  const float total = sf_wave_sum(part);
  int key[J];
#pragma unroll
  for (int j = 0; j < J; ++j) key[j] = lane + SF_WAVE * j < E ? __float_as_int(x[j] / total) : -1;
  float mine = 0.0f;
  int mine_id = 0;
  for (int r = 0; r < K; ++r) {
    int lk = key[0];
#pragma unroll
    for (int j = 1; j < J; ++j) lk = max(lk, key[j]);
    const int bk = sf_wave_max_int(lk);
    int be = -1;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const unsigned long long hit = __ballot(key[j] == bk);
      if (be < 0 && hit) be = SF_WAVE * j + __ffsll(hit) - 1;
    }
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (be == lane + SF_WAVE * j) key[j] = -1;
    if (lane == r) {
      mine = __int_as_float(bk);
      mine_id = be;
    }
  }
  float sum = 0.0f;
  if (renorm)
    for (int r = 0; r < K; ++r) sum += sf_readlane(mine, r);
  if (lane < K) {
    const float v = renorm ? mine / sum : mine;
    topw[lane] = sf_f32_to_bf16(v);
    topi[lane] = static_cast<int64_t>(mine_id);
  }
}

// Vector path: hidden_size % 8 == 0, 16-byte aligned rows and at most NCH
// chunks of 8 elements per lane.  Two kernels, so the dot products spread
// over the whole chip: the logits kernel gives each wavefront a tile of TT
// tokens x EPW experts (all loads of the tile issued before any use, each
// logit summed per lane and butterflied exactly as above), the select
// kernel runs softmax / top-k / renormalisation with one wavefront per
// token.
constexpr int kLogitWaves = 4;
template <int NCH>
struct LogitTile {
  static constexpr int experts = NCH <= 4 ? 4 : (NCH <= 8 ? 2 : 1);  // per wavefront
  static constexpr int tokens = NCH <= 4 ? 2 : 1;
};

template <int NCH>
__global__ __launch_bounds__(kLogitWaves * SF_WAVE) void router_logits_kernel(
    const uint16_t* __restrict__ hidden, const uint16_t* __restrict__ wr, int T, int H,
    int E, uint16_t* __restrict__ logits) {
  constexpr int EPW = LogitTile<NCH>::experts;
  constexpr int TT = LogitTile<NCH>::tokens;
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int t0 = blockIdx.x * TT;
  const int e0 = (blockIdx.y * kLogitWaves + wave) * EPW;
  if (e0 >= E) return;  // wave-uniform; the kernel has no block barrier
  const int nchunks = H / 8;
  uint4 hreg[TT][NCH];
  uint4 wv[EPW][NCH];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    const uint4* h4 =
        reinterpret_cast<const uint4*>(hidden + static_cast<size_t>(min(t0 + tt, T - 1)) * H);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + SF_WAVE * i;
      hreg[tt][i] = c < nchunks ? h4[c] : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int g = 0; g < EPW; ++g) {
    const uint4* w4 = reinterpret_cast<const uint4*>(wr + static_cast<size_t>(min(e0 + g, E - 1)) * H);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + SF_WAVE * i;
      wv[g][i] = c < nchunks ? w4[c] : make_uint4(0, 0, 0, 0);
    }
  }
  float acc[TT][EPW];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int g = 0; g < EPW; ++g) {
      acc[tt][g] = 0.0f;
#pragma unroll
      for (int i = 0; i < NCH; ++i)
        if (lane + SF_WAVE * i < nchunks) acc[tt][g] = dot8_acc(hreg[tt][i], wv[g][i], acc[tt][g]);
    }
  // Lane tt*EPW + g stores logit (t0+tt, e0+g).
  float a = 0.0f;
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int g = 0; g < EPW; ++g) {
      const float total = sf_wave_sum(acc[tt][g]);
      if (lane == tt * EPW + g) a = total;
    }
  const int t = t0 + lane / EPW;
  const int e = e0 + lane % EPW;
  if (lane < TT * EPW && t < T && e < E)
    logits[static_cast<size_t>(t) * E + e] = sf_f32_to_bf16(a);
}

constexpr int kSelectWaves = 4;

template <int J>  // experts per lane: E <= 64 * J
__global__ __launch_bounds__(kSelectWaves * SF_WAVE) void router_select_kernel(
    const uint16_t* __restrict__ logits, int T, int E, int K, int renorm,
    uint16_t* __restrict__ topw, int64_t* __restrict__ topi) {
  __shared__ float s_logit[kSelectWaves][SF_MAX_EXPERTS];
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int t = blockIdx.x * kSelectWaves + wave;
  if (t >= T) return;  // wave-uniform; the kernel has no block barrier
  // Lane l writes and later reads only experts l, l+64, ...: no barrier.
  for (int e = lane; e < E; e += SF_WAVE)
    s_logit[wave][e] = sf_bf16_to_f32(logits[static_cast<size_t>(t) * E + e]);
  softmax_topk_wave<J>(s_logit[wave], E, K, renorm, topw + static_cast<size_t>(t) * K,
                       topi + static_cast<size_t>(t) * K);
}

// Scalar path for any hidden_size / alignment: same summation order.
__global__ __launch_bounds__(kRouterThreads) void router_topk_scalar_kernel(
    const uint16_t* __restrict__ hidden, const uint16_t* __restrict__ wr, int H,
    int E, int K, int renorm, uint16_t* __restrict__ logits,
    uint16_t* __restrict__ topw, int64_t* __restrict__ topi) {
  __shared__ float s_logit[SF_MAX_EXPERTS];
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
    acc = sf_wave_sum(acc);
    if (lane == 0) {
      uint16_t b = sf_f32_to_bf16(acc);
      logits[static_cast<size_t>(t) * E + e] = b;
      s_logit[e] = sf_bf16_to_f32(b);
    }
  }
  __syncthreads();
  if (wave == 0)
    softmax_topk_wave<SF_MAX_EXPERTS / SF_WAVE>(s_logit, E, K, renorm,
                                                topw + static_cast<size_t>(t) * K,
                                                topi + static_cast<size_t>(t) * K);
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
  if (aligned && per_lane <= 16) {
    int tt = 1, epw = 1;
    auto logits_launch = [&](auto kernel, int tile_tokens, int tile_experts) {
      tt = tile_tokens;
      epw = tile_experts;
      const int per_block = kLogitWaves * epw;
      dim3 grid((tokens + tt - 1) / tt, (num_experts + per_block - 1) / per_block);
      kernel<<<grid, dim3(kLogitWaves * SF_WAVE), 0, s>>>(h, w, tokens, hidden_size, num_experts, lg);
    };
    if (per_lane <= 1)
      logits_launch(router_logits_kernel<1>, LogitTile<1>::tokens, LogitTile<1>::experts);
    else if (per_lane <= 2)
      logits_launch(router_logits_kernel<2>, LogitTile<2>::tokens, LogitTile<2>::experts);
    else if (per_lane <= 4)
      logits_launch(router_logits_kernel<4>, LogitTile<4>::tokens, LogitTile<4>::experts);
    else if (per_lane <= 8)
      logits_launch(router_logits_kernel<8>, LogitTile<8>::tokens, LogitTile<8>::experts);
    else
      logits_launch(router_logits_kernel<16>, LogitTile<16>::tokens, LogitTile<16>::experts);
    SF_LAUNCH_CHECK();
    // Experts per lane of the select wavefront: dead slots (e >= E) add +0
    // to the lane sums and are never selected, so J only trims the loops.
    const dim3 sgrid((tokens + kSelectWaves - 1) / kSelectWaves), sblock(kSelectWaves * SF_WAVE);
    if (num_experts <= SF_WAVE)
      router_select_kernel<1><<<sgrid, sblock, 0, s>>>(lg, tokens, num_experts, top_k,
                                                       norm_topk_prob, tw, topk_index);
    else if (num_experts <= 2 * SF_WAVE)
      router_select_kernel<2><<<sgrid, sblock, 0, s>>>(lg, tokens, num_experts, top_k,
                                                       norm_topk_prob, tw, topk_index);
    else
      router_select_kernel<SF_MAX_EXPERTS / SF_WAVE><<<sgrid, sblock, 0, s>>>(
          lg, tokens, num_experts, top_k, norm_topk_prob, tw, topk_index);
  } else {
    router_topk_scalar_kernel<<<dim3(tokens), dim3(kRouterThreads), 0, s>>>(
        h, w, hidden_size, num_experts, top_k, norm_topk_prob, lg, tw, topk_index);
  }
  SF_LAUNCH_CHECK();
  return SF_OK;
}
