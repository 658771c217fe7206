// K4: deterministic weighted combine (gather + add) in a fixed expert order.
// Restates zeros_like + index_add_ of the per-expert contributions of the
// reference (src/specfit/runtime/qwen3_offloaded_experts.py:144-164,
// 200-202).  K3 already scaled every row by its routing weight, so the
// combine only sums, per token, the rows of its routes.  The routes of a token
// are visited in ascending (expert_rank[expert], position) order: canonical
// mode ranks experts by id, arrival-order mode by execution order.  With bf16
// accumulation each addition is rounded to bf16, which is what a sequence of
// bf16 index_add_ calls computes; no atomics, so the result is bitwise
// reproducible.
#include "sf_common.h"

namespace {

constexpr int kCombineThreads = 256;
constexpr int kColsPerThread = 8;
constexpr int kColsPerBlock = kCombineThreads * kColsPerThread;

struct RankTable {
  int32_t rank[SF_MAX_EXPERTS];
};

__device__ __forceinline__ void unpack8(uint4 q, uint16_t* v) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    v[2 * c] = static_cast<uint16_t>(w[c] & 0xffffu);
    v[2 * c + 1] = static_cast<uint16_t>(w[c] >> 16);
  }
}

// One block per (token, 2048-column slice).  Threads 0..K-1 fetch the
// token's routes in parallel and each places its route at its rank in
// (key, position) order (the routes ordered before it, counted in LDS).  Up to
// kPrefetch rows are then loaded before any addition so the gather costs one
// memory round trip, and the additions run in the fixed order.
constexpr int kPrefetch = 8;

template <bool kVec>
__global__ __launch_bounds__(kCombineThreads) void combine_kernel(
    const uint16_t* __restrict__ rows, const int64_t* __restrict__ idx,
    const int32_t* __restrict__ inv_perm, const RankTable ranks, int use_rank,
    int K, int E, int H, int acc_fp32, uint16_t* __restrict__ out) {
  __shared__ int s_key[SF_MAX_TOPK];
  __shared__ int s_rowid[SF_MAX_TOPK];
  __shared__ int s_row[SF_MAX_TOPK];
  __shared__ int s_n;
  const int t = blockIdx.x;
  if (threadIdx.x < K) {
    const int j = threadIdx.x;
    const int64_t e = idx[static_cast<int64_t>(t) * K + j];
    const int r = inv_perm[static_cast<int64_t>(t) * K + j];
    const bool ok = e >= 0 && e < E && r >= 0;
    s_key[j] = ok ? (use_rank ? ranks.rank[e] : static_cast<int>(e)) : -1;
    s_rowid[j] = ok ? r : -1;
  }
  __syncthreads();
  if (threadIdx.x < K) {
    // Stable order on (key, position): a route's slot is the number of
    // valid routes with a smaller key, or an equal key at an earlier position.
    const int j = threadIdx.x;
    const int row = s_rowid[j];
    const int k = s_key[j];
    int pos = 0, n = 0;
    for (int i = 0; i < K; ++i) {
      if (s_rowid[i] < 0) continue;
      ++n;
      const int ki = s_key[i];
      pos += (ki < k) || (ki == k && i < j);
    }
    if (row >= 0) s_row[pos] = row;
    if (j == 0) s_n = n;
  }
  __syncthreads();
  const int c0 = blockIdx.y * kColsPerBlock + threadIdx.x * kColsPerThread;
  if (c0 >= H) return;
  const int n = s_n;
  float acc[kColsPerThread];
#pragma unroll
  for (int c = 0; c < kColsPerThread; ++c) acc[c] = 0.0f;
  for (int j0 = 0; j0 < n; j0 += kPrefetch) {
    uint16_t v[kPrefetch][kColsPerThread];
#pragma unroll
    for (int j = 0; j < kPrefetch; ++j) {
      if (j0 + j < n) {
        const uint16_t* src = rows + static_cast<int64_t>(s_row[j0 + j]) * H + c0;
        if (kVec) {
          unpack8(*reinterpret_cast<const uint4*>(src), v[j]);
        } else {
#pragma unroll
          for (int c = 0; c < kColsPerThread; ++c) v[j][c] = c0 + c < H ? src[c] : 0;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kPrefetch; ++j) {
      if (j0 + j < n) {
#pragma unroll
        for (int c = 0; c < kColsPerThread; ++c) {
          const float s = acc[c] + sf_bf16_to_f32(v[j][c]);
          acc[c] = acc_fp32 ? s : sf_round_bf16(s);
        }
      }
    }
  }
  uint16_t* dst = out + static_cast<int64_t>(t) * H + c0;
  if (kVec) {
    uint32_t w[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      w[c] = static_cast<uint32_t>(sf_f32_to_bf16(acc[2 * c])) |
             (static_cast<uint32_t>(sf_f32_to_bf16(acc[2 * c + 1])) << 16);
    *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
#pragma unroll
    for (int c = 0; c < kColsPerThread; ++c)
      if (c0 + c < H) dst[c] = sf_f32_to_bf16(acc[c]);
  }
}

}  // namespace

extern "C" int sf_combine(const void* rows, const int64_t* topk_index,
                          const int32_t* inv_perm, const int32_t* expert_rank,
                          int tokens, int top_k, int num_experts, int hidden_size,
                          int accumulate_fp32, void* out, sf_stream_t stream) {
  if (tokens < 0 || top_k < 1 || top_k > SF_MAX_TOPK || num_experts < 1 ||
      num_experts > SF_MAX_EXPERTS || hidden_size < 1)
    return SF_ERR_INVALID_ARGUMENT;
  if (tokens == 0) return SF_OK;
  if (!rows || !topk_index || !inv_perm || !out) return SF_ERR_INVALID_ARGUMENT;
  RankTable ranks{};
  if (expert_rank)
    for (int e = 0; e < num_experts; ++e) ranks.rank[e] = expert_rank[e];
  const bool vec = hidden_size % 8 == 0 && (reinterpret_cast<uintptr_t>(rows) & 15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
  dim3 grid(tokens, (hidden_size + kColsPerBlock - 1) / kColsPerBlock);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (vec)
    combine_kernel<true><<<grid, kCombineThreads, 0, s>>>(
        static_cast<const uint16_t*>(rows), topk_index, inv_perm, ranks,
        expert_rank != nullptr, top_k, num_experts, hidden_size, accumulate_fp32,
        static_cast<uint16_t*>(out));
  else
    combine_kernel<false><<<grid, kCombineThreads, 0, s>>>(
        static_cast<const uint16_t*>(rows), topk_index, inv_perm, ranks,
        expert_rank != nullptr, top_k, num_experts, hidden_size, accumulate_fp32,
        static_cast<uint16_t*>(out));
  SF_LAUNCH_CHECK();
  return SF_OK;
}
