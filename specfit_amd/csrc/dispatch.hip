// K2: token-to-expert dispatch as a stable counting sort in LDS.
// Restates the stable sort of the flattened routes by expert id plus
// unique_consecutive / route_tokens of the reference
// (src/specfit/runtime/qwen3_offloaded_experts.py:173-178).
//
// One workgroup walks the N = tokens*top_k route positions in chunks of its
// thread count.  Per chunk every wavefront ranks its lanes among equal
// expert ids with a ballot loop (rank = lanes below with the same id), the
// per-wavefront counts are prefix-summed per expert in wavefront order, and
// each route lands at offsets[e] + (routes of e in earlier chunks) +
// (routes of e in earlier wavefronts) + rank.  This is exactly the ascending
// position order inside every expert, i.e. a stable sort.
#include "sf_common.h"

namespace {

// One workgroup of kDispatchThreads (1024, or 256 when the routes fit one
// 256-wide chunk: fewer wavefronts to synchronise).  The permutation is the
// unique stable order either way.
template <int kDispatchThreads>
__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(
    const int64_t* __restrict__ idx, int N, int E, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm_pos,
    int32_t* __restrict__ inv_perm, int32_t* __restrict__ host_meta) {
  constexpr int kDispatchWaves = kDispatchThreads / SF_WAVE;
  __shared__ int s_total[SF_MAX_EXPERTS];
  __shared__ int s_offset[SF_MAX_EXPERTS + 1];
  __shared__ int s_running[SF_MAX_EXPERTS];
  __shared__ int s_wave_count[kDispatchWaves][SF_MAX_EXPERTS];
  __shared__ int s_invalid;
  const int tid = threadIdx.x;
  const int lane = tid & (SF_WAVE - 1);
  const int wave = tid / SF_WAVE;

  for (int e = tid; e < SF_MAX_EXPERTS; e += kDispatchThreads) {
    s_total[e] = 0;
    s_running[e] = 0;
  }
  for (int i = tid; i < kDispatchWaves * SF_MAX_EXPERTS; i += kDispatchThreads)
    (&s_wave_count[0][0])[i] = 0;
  if (tid == 0) s_invalid = 0;
  __syncthreads();

  // Pass 1: histogram (integer atomics are order independent).  Each
  // thread keeps its first id (position tid) for the first scatter chunk.
  int64_t first = -1;
  for (int i = tid; i < N; i += kDispatchThreads) {
    int64_t e = idx[i];
    if (i == tid) first = e;
    if (e >= 0 && e < E)
      atomicAdd(&s_total[e], 1);
    else
      atomicAdd(&s_invalid, 1);
  }
  __syncthreads();
  if (wave == 0) {
    // Exclusive prefix of s_total over the experts: lane l owns experts
    // 4l .. 4l+3 (SF_MAX_EXPERTS = 256 = 4 x 64), a wavefront inclusive scan
    // of the lane sums gives each lane its starting offset.
    constexpr int kPer = SF_MAX_EXPERTS / SF_WAVE;
    int own[kPer];
    int sum = 0;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int e = lane * kPer + q;
      own[q] = e < E ? s_total[e] : 0;
      sum += own[q];
    }
    int incl = sum;
#pragma unroll
    for (int d = 1; d < SF_WAVE; d <<= 1) {
      const int up = __shfl_up(incl, d, SF_WAVE);
      if (lane >= d) incl += up;
    }
    int run = incl - sum;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int e = lane * kPer + q;
      if (e < E) s_offset[e] = run;
      run += own[q];
    }
    if (lane == SF_WAVE - 1) s_offset[E] = incl;
  }
  __syncthreads();
  for (int e = tid; e < E; e += kDispatchThreads) {
    counts[e] = s_total[e];
    offsets[e] = s_offset[e];
  }
  if (tid == 0) {
    counts[E] = s_invalid;
    offsets[E] = s_offset[E];
  }
  if (host_meta) {  // the same [counts; offsets] into pinned host memory
    for (int e = tid; e < E; e += kDispatchThreads) {
      host_meta[e] = s_total[e];
      host_meta[E + 1 + e] = s_offset[e];
    }
    if (tid == 0) {
      host_meta[E] = s_invalid;
      host_meta[2 * E + 1] = s_offset[E];
    }
  }

  // Pass 2: stable scatter, chunk by chunk.
  for (int base = 0; base < N; base += kDispatchThreads) {
    const int i = base + tid;
    int e = -1;
    if (i < N) {
      const int64_t v = base == 0 ? first : idx[i];
      e = (v >= 0 && v < E) ? static_cast<int>(v) : -1;
    }
    // One round per distinct id of the wavefront: the lowest pending lane
    // leads, its id is read with a scalar lane read (no LDS round trip on
    // the loop's dependency chain), and the lanes holding it take their
    // rank (lanes below with the same id, mbcnt) and group size.
    int rank = 0, group = 0;
    uint64_t pending = __ballot(e >= 0);
    while (pending) {
      const int leader = __ffsll(static_cast<unsigned long long>(pending)) - 1;
      const int le = __builtin_amdgcn_readlane(e, leader);
      const uint64_t same = __ballot(e == le);
      if (e == le) {
        rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(same >> 32),
                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(same), 0));
        group = __popcll(same);
      }
      pending &= ~same;
    }
    const bool valid = e >= 0;
    if (valid && rank == 0) s_wave_count[wave][e] = group;
    __syncthreads();
    // Exclusive prefix over the wavefronts that hold routes in this chunk
    // (the others' counts are zero), per expert, continuing the running
    // count of earlier chunks.
    const int busy_waves = min(kDispatchWaves, (min(N - base, kDispatchThreads) + SF_WAVE - 1) / SF_WAVE);
    for (int ex = tid; ex < E; ex += kDispatchThreads) {
      int run = s_running[ex];
      for (int w = 0; w < busy_waves; ++w) {
        int c = s_wave_count[w][ex];
        s_wave_count[w][ex] = run;
        run += c;
      }
      s_running[ex] = run;
    }
    __syncthreads();
    if (i < N) {
      if (valid) {
        const int pos = s_offset[e] + s_wave_count[wave][e] + rank;
        perm_pos[pos] = i;
        inv_perm[i] = pos;
      } else {
        inv_perm[i] = -1;
      }
    }
    if (base + kDispatchThreads >= N) break;  // last chunk: nothing to reset
    __syncthreads();
    // Reset the per-wavefront table for the next chunk.
    for (int j = tid; j < kDispatchWaves * SF_MAX_EXPERTS; j += kDispatchThreads)
      (&s_wave_count[0][0])[j] = 0;
    __syncthreads();
  }
}

}  // namespace

extern "C" int sf_dispatch(const int64_t* topk_index, int tokens, int top_k,
                           int num_experts, int32_t* counts, int32_t* offsets,
                           int32_t* perm_pos, int32_t* inv_perm, int32_t* host_meta,
                           sf_stream_t stream) {
  if (tokens < 0 || top_k < 1 || num_experts < 1 || num_experts > SF_MAX_EXPERTS)
    return SF_ERR_INVALID_ARGUMENT;
  const long long n = static_cast<long long>(tokens) * top_k;
  if (n > 0x7fffffffLL) return SF_ERR_UNSUPPORTED_SHAPE;
  if (!counts || !offsets) return SF_ERR_INVALID_ARGUMENT;
  if (n > 0 && (!topk_index || !perm_pos || !inv_perm)) return SF_ERR_INVALID_ARGUMENT;
  int32_t* host_dev = nullptr;  // the device's address of host_meta
  if (host_meta) {
    void* p = nullptr;
    if (hipHostGetDevicePointer(&p, host_meta, 0) != hipSuccess || !p)
      return SF_ERR_INVALID_ARGUMENT;
    host_dev = static_cast<int32_t*>(p);
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (n <= 256)
    dispatch_kernel<256><<<1, 256, 0, s>>>(topk_index, static_cast<int>(n), num_experts, counts,
                                           offsets, perm_pos, inv_perm, host_dev);
  else
    dispatch_kernel<1024><<<1, 1024, 0, s>>>(topk_index, static_cast<int>(n), num_experts, counts,
                                             offsets, perm_pos, inv_perm, host_dev);
  SF_LAUNCH_CHECK();
  return SF_OK;
}
