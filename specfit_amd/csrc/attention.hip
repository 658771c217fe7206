// K5: tree-verification attention (grouped-query) on gfx950.
//
// Replaces the attention the target model runs in the verification forward
// (src/specfit/runtime/eagle3_tree.py:1202-1240 calls the HF target with the
// draft tree's mask; Qwen3MoeAttention then runs sdpa_attention_forward of
// transformers/integrations/sdpa_attention.py with that 4-D bool mask).
// For query token qi, query head qh = h*G + j of key/value head h:
//   out[qi, qh] = sum_s softmax_s(scale * q[qi, qh] . k[h, s]) * v[h, s]
// over keys s the mask admits (mask[qi, s] != 0; with no mask, s <= S - Q + qi,
// i.e. causal aligned to the end of the keys).  A query with no admitted key
// gets 0.
//
// At verification sizes (Q = 61 tree tokens, S ~ 1.1k keys, 32 query heads,
// 4 KV heads, head dim 128) the whole layer's K/V is ~2 MB: the kernel is
// latency-bound, not HBM-bound.  One workgroup per (query, KV head) keeps the
// G query heads of the group together so each K/V row is read once per
// query.  Its 4 wavefronts take interleaved 64-key chunks: scores with one
// key per lane (the query rows broadcast from LDS), an online softmax per
// head across the wavefront, then P.V with one value row per step and the
// head-dim elements spread over the lanes.  The four partial (max, sum,
// accumulator) states are merged in wavefront order, so the fp32 summation
// order is fixed and results are run-to-run identical.
#include "sf_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / SF_WAVE;
constexpr int kChunk = SF_WAVE;  // keys per wavefront chunk

struct AttnArgs {
  const uint16_t* q;
  int64_t q_tok, q_head;
  const uint16_t* k;
  int64_t k_head, k_tok;
  const uint16_t* v;
  int64_t v_head, v_tok;
  const uint8_t* mask;  // nullptr: causal aligned to the end
  int64_t mask_q;
  int Q, S, Hkv, D;
  float scale;
  uint16_t* out;  // [Q, Hkv * G, D]
};

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, SF_WAVE));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, SF_WAVE);
  return x;
}

// G query heads per KV head; DPL head-dim elements per lane in P.V (D <= 64*DPL).
template <int G, int DPL>
__global__ __launch_bounds__(kThreads) void tree_attention_kernel(const AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int D = a.D;
  float* sq = smem;                                 // [G][D] scaled query rows
  float* sp = sq + G * D;                           // [kWaves][G][kChunk] probabilities
  float* sm = sp + kWaves * G * kChunk;             // [kWaves][G] running max
  float* sl = sm + kWaves * G;                      // [kWaves][G] running sum
  float* sacc = sl + kWaves * G;                    // [kWaves][G][D] accumulators
  const int qi = blockIdx.x / a.Hkv;
  const int h = blockIdx.x - qi * a.Hkv;
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;

  for (int i = threadIdx.x; i < G * D; i += kThreads) {
    const int j = i / D;
    const int d = i - j * D;
    sq[i] = sf_bf16_to_f32(a.q[qi * a.q_tok + static_cast<int64_t>(h * G + j) * a.q_head + d]) *
            a.scale;
  }
  __syncthreads();

  const uint16_t* kh = a.k + h * a.k_head;
  const uint16_t* vh = a.v + h * a.v_head;
  const int causal_last = a.S - a.Q + qi;  // last admitted key without a mask
  float m[G], l[G], acc[G][DPL];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[j][e] = 0.f;
  }
  float* pw = sp + wave * G * kChunk;
  const int d0 = lane * DPL;

  for (int kb = wave * kChunk; kb < a.S; kb += kWaves * kChunk) {
    // Scores: lane -> key kb + lane.
    const int key = kb + lane;
    bool ok = key < a.S;
    if (ok) ok = a.mask ? a.mask[qi * a.mask_q + key] != 0 : key <= causal_last;
    float s[G];
#pragma unroll
    for (int j = 0; j < G; ++j) s[j] = 0.f;
    if (ok) {
      const uint16_t* kr = kh + key * a.k_tok;
      for (int d = 0; d < D; d += 8) {
        const uint4 kv = *reinterpret_cast<const uint4*>(kr + d);
        float kf[8];
        const uint32_t w[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kf[2 * e] = __uint_as_float(w[e] << 16);
          kf[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
        }
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const float* qr = sq + j * D + d;
#pragma unroll
          for (int e = 0; e < 8; ++e) s[j] = __builtin_fmaf(qr[e], kf[e], s[j]);
        }
      }
    }
    // Online softmax per head over this chunk.
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float cmax = wave_max(ok ? s[j] : -INFINITY);
      const float mnew = fmaxf(m[j], cmax);
      float p = 0.f;
      float alpha = 1.f;
      if (mnew != -INFINITY) {
        alpha = m[j] == -INFINITY ? 0.f : __expf(m[j] - mnew);
        if (ok) p = __expf(s[j] - mnew);
      }
      l[j] = l[j] * alpha + wave_sum(p);
      m[j] = mnew;
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[j][e] *= alpha;
      pw[j * kChunk + lane] = p;
    }
    // P.V: one value row per step, head-dim elements d0 .. d0+DPL-1 per lane.
    const int nkeys = min(kChunk, a.S - kb);
    if (d0 < D) {
      for (int t = 0; t < nkeys; ++t) {
        const uint16_t* vr = vh + (kb + t) * a.v_tok + d0;
        float vf[DPL];
#pragma unroll
        for (int e = 0; e < DPL; ++e) vf[e] = sf_bf16_to_f32(vr[e]);
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const float p = pw[j * kChunk + t];
#pragma unroll
          for (int e = 0; e < DPL; ++e) acc[j][e] = __builtin_fmaf(p, vf[e], acc[j][e]);
        }
      }
    }
  }

  // Merge the wavefront states in wavefront order.
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < G; ++j) {
      sm[wave * G + j] = m[j];
      sl[wave * G + j] = l[j];
    }
  }
  if (d0 < D) {
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int e = 0; e < DPL; ++e) sacc[(wave * G + j) * D + d0 + e] = acc[j][e];
  }
  __syncthreads();
  const int Hq = a.Hkv * G;
  for (int i = threadIdx.x; i < G * D; i += kThreads) {
    const int j = i / D;
    const int d = i - j * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm[w * G + j]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float mw = sm[w * G + j];
        if (mw == -INFINITY) continue;
        const float f = __expf(mw - M);
        L = __builtin_fmaf(sl[w * G + j], f, L);
        O = __builtin_fmaf(sacc[(w * G + j) * D + d], f, O);
      }
    }
    const float o = L > 0.f ? O / L : 0.f;
    a.out[(static_cast<int64_t>(qi) * Hq + h * G + j) * D + d] = sf_f32_to_bf16(o);
  }
}

// LDS bytes of one workgroup: query rows, chunk probabilities, merge state.
size_t lds_bytes(int G, int D) {
  return sizeof(float) * (static_cast<size_t>(G) * D + kWaves * G * kChunk + 2 * kWaves * G +
                          static_cast<size_t>(kWaves) * G * D);
}

constexpr size_t kMaxLds = 64 * 1024;

template <int G>
int launch_g(const AttnArgs& a, hipStream_t s) {
  const int dpl = (a.D + SF_WAVE - 1) / SF_WAVE;
  const size_t lds = lds_bytes(G, a.D);
  const dim3 grid(static_cast<unsigned>(a.Q) * a.Hkv);
  if (dpl == 1)
    tree_attention_kernel<G, 1><<<grid, kThreads, lds, s>>>(a);
  else if (dpl == 2)
    tree_attention_kernel<G, 2><<<grid, kThreads, lds, s>>>(a);
  else
    tree_attention_kernel<G, 4><<<grid, kThreads, lds, s>>>(a);
  SF_LAUNCH_CHECK();
  return SF_OK;
}

bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

}  // namespace

extern "C" int sf_tree_attention(const void* q, int64_t q_stride_token, int64_t q_stride_head,
                                 const void* k, int64_t k_stride_head, int64_t k_stride_token,
                                 const void* v, int64_t v_stride_head, int64_t v_stride_token,
                                 const uint8_t* mask, int64_t mask_stride_query, int queries,
                                 int keys, int q_heads, int kv_heads, int head_dim, float scale,
                                 void* out, sf_stream_t stream) {
  if (queries < 1 || keys < 1 || q_heads < 1 || kv_heads < 1 || head_dim < 1)
    return SF_ERR_INVALID_ARGUMENT;
  if (!q || !k || !v || !out) return SF_ERR_INVALID_ARGUMENT;
  if (q_heads % kv_heads) return SF_ERR_UNSUPPORTED_SHAPE;
  const int G = q_heads / kv_heads;
  if (head_dim % 8 || head_dim > 4 * SF_WAVE) return SF_ERR_UNSUPPORTED_SHAPE;
  if (lds_bytes(G, head_dim) > kMaxLds) return SF_ERR_UNSUPPORTED_SHAPE;
  if (static_cast<long long>(queries) * kv_heads > 0x7fffffffLL) return SF_ERR_UNSUPPORTED_SHAPE;
  if (q_stride_token < 0 || q_stride_head < 0 || k_stride_head < 0 || v_stride_head < 0 ||
      k_stride_token < head_dim || v_stride_token < head_dim ||
      (mask && mask_stride_query < keys))
    return SF_ERR_INVALID_ARGUMENT;
  // Key rows are read 16 B at a time; value rows DPL elements per lane.
  const int dpl = (head_dim + SF_WAVE - 1) / SF_WAVE;
  if (!aligned(k, 16) || k_stride_token % 8 || k_stride_head % 8) return SF_ERR_MISALIGNED;
  const int dpl_bytes = dpl * 2;
  if (!aligned(v, dpl_bytes) || (v_stride_token * 2) % dpl_bytes || (v_stride_head * 2) % dpl_bytes)
    return SF_ERR_MISALIGNED;
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_tok = q_stride_token;
  a.q_head = q_stride_head;
  a.k = static_cast<const uint16_t*>(k);
  a.k_head = k_stride_head;
  a.k_tok = k_stride_token;
  a.v = static_cast<const uint16_t*>(v);
  a.v_head = v_stride_head;
  a.v_tok = v_stride_token;
  a.mask = mask;
  a.mask_q = mask_stride_query;
  a.Q = queries;
  a.S = keys;
  a.Hkv = kv_heads;
  a.D = head_dim;
  a.scale = scale;
  a.out = static_cast<uint16_t*>(out);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (G) {
    case 1: return launch_g<1>(a, s);
    case 2: return launch_g<2>(a, s);
    case 4: return launch_g<4>(a, s);
    case 8: return launch_g<8>(a, s);
    case 16: return launch_g<16>(a, s);
    default: return SF_ERR_UNSUPPORTED_SHAPE;
  }
}
