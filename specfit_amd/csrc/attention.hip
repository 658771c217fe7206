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
// latency-bound, not HBM-bound.  Head dims 64 and 128 with 2..16 query heads
// per KV head run the MFMA form below (26 us at the 61-token verification
// shape and 28 us at 128 tokens on MI355X, against 54 and 108 us for the
// loop form).  The loop form covers every other shape: one workgroup per
// (query, KV head) keeps the
// G query heads of the group together so each K/V row is read once per
// query.  Its 8 wavefronts take interleaved 64-key chunks: scores with one
// key per lane (the key row in registers, the query rows broadcast from
// LDS), an online softmax per head across the wavefront, then P.V with the
// head-dim elements spread over the lanes and the value rows of 16 keys
// loaded together.  The eight partial (max, sum, accumulator) states are
// merged in wavefront order, so the fp32 summation order is fixed and
// results are run-to-run identical.
#include "sf_common.h"

namespace {

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

// x plus the value of lane `CTRL`-permuted lane (a DPP move: no LDS).
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
  const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false);
  return x + __int_as_float(moved);
}

// Sum over aligned groups of N lanes (N = 8 or 16), every lane gets it:
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  x = dpp_add<0xB1>(x);
  x = dpp_add<0x4E>(x);
  x = dpp_add<0x141>(x);
  if (N == 16) x = dpp_add<0x140>(x);
  return x;
}

__device__ __forceinline__ void unpack8(const uint4 v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(w[e] << 16);
    f[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
}

// G query heads per KV head.  DC > 0: head dim 8*DC known at compile time
// (every loop unrolled, a chunk's key and value loads issued together);
// DC == 0: any head dim (multiple of 8, <= 256) read from the arguments.
// DPL head-dim elements per lane in P.V.  NW wavefronts per workgroup.
template <int G, int DC, int DPL, int NW>
__global__ __launch_bounds__(NW * SF_WAVE) void tree_attention_kernel(const AttnArgs a) {
  constexpr int kWaves = NW;
  constexpr int kThreads = NW * SF_WAVE;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int D = DC > 0 ? 8 * DC : a.D;
  float* sq = smem;                                 // [G][D] scaled query rows
  float* sm = sq + G * D;                           // [kWaves][G] running max
  float* sl = sm + kWaves * G;                      // [kWaves][G] running sum
  float* sp = sl + kWaves * G;                      // [kWaves][G][kChunk] probabilities
  float* sacc = sp;                                 // [kWaves][G][D] accumulators (after
                                                    // the key loop, over sp)
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
  // Compile-time head dim: this lane's 8 query elements of every head.
  float qreg[DC > 0 ? G : 1][8];
  if (DC > 0) {
    const int dc = lane % (DC > 0 ? DC : 1);
#pragma unroll
    for (int j = 0; j < (DC > 0 ? G : 1); ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) qreg[j][e] = sq[j * D + 8 * dc + e];
  }
  const bool has_d = d0 < D;

  for (int kb = wave * kChunk; kb < a.S; kb += kWaves * kChunk) {
    const int nkeys = min(kChunk, a.S - kb);
    // Scores.  With the head dim known (DC > 0), DC lanes share one key: lane
    // l holds query elements 8*(l%DC) .. +7 of every head in registers,
    // multiplies them with its 16 B of the key row and the DC partial sums
    // are added by a butterfly; the chunk's scores go through LDS to the
    // one-key-per-lane layout of the softmax.  Otherwise lane -> key.
    const int key = kb + lane;
    bool ok = key < a.S;
    if (ok) ok = a.mask ? a.mask[qi * a.mask_q + key] != 0 : key <= causal_last;
    float s[G];
    if (DC > 0) {
      constexpr int kKeysPer = DC > 0 ? SF_WAVE / DC : 1;  // keys per instruction
      constexpr int kIters = kChunk / kKeysPer;
      const int kq = lane / (DC > 0 ? DC : 1);
      const int dc = lane % (DC > 0 ? DC : 1);
      uint4 kv[kIters];
#pragma unroll
      for (int i = 0; i < kIters; ++i) {
        const int kk = min(kb + i * kKeysPer + kq, a.S - 1);
        kv[i] = *reinterpret_cast<const uint4*>(kh + kk * a.k_tok + 8 * dc);
      }
#pragma unroll
      for (int i = 0; i < kIters; ++i) {
        float kf[8];
        unpack8(kv[i], kf);
#pragma unroll
        for (int j = 0; j < G; ++j) {
          float part = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) part = __builtin_fmaf(qreg[j][e], kf[e], part);
          part = group_sum<(DC == 16 ? 16 : 8)>(part);
          if (dc == 0) pw[j * kChunk + i * kKeysPer + kq] = part;
        }
      }
#pragma unroll
      for (int j = 0; j < G; ++j) s[j] = pw[j * kChunk + lane];
    } else {
#pragma unroll
      for (int j = 0; j < G; ++j) s[j] = 0.f;
      const uint16_t* kr = kh + min(key, a.S - 1) * a.k_tok;
      for (int d = 0; d < D; d += 8) {
        float kf[8];
        unpack8(*reinterpret_cast<const uint4*>(kr + d), kf);
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
    // P.V: head-dim elements d0 .. d0+DPL-1 per lane; the value rows of a
    // group of 16 keys are loaded together, then accumulated.
    if (has_d) {
      const uint16_t* vc = vh + kb * a.v_tok + d0;
      for (int t0 = 0; t0 < nkeys; t0 += 16) {
        float vf[16][DPL];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          const uint16_t* vr = vc + min(t0 + t, nkeys - 1) * a.v_tok;
#pragma unroll
          for (int e = 0; e < DPL; ++e) vf[t][e] = sf_bf16_to_f32(vr[e]);
        }
        // Keys past the end carry p = 0 (and a finite repeated row).
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const float4* p4 = reinterpret_cast<const float4*>(pw + j * kChunk + t0);
#pragma unroll
          for (int t4 = 0; t4 < 4; ++t4) {
            const float4 p = p4[t4];
            const float pp[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
              for (int e = 0; e < DPL; ++e)
                acc[j][e] = __builtin_fmaf(pp[u], vf[4 * t4 + u][e], acc[j][e]);
          }
        }
      }
    }
  }

  // Merge the wavefront states in wavefront order.
  __syncthreads();  // every wavefront is done with sp, which sacc overlays
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < G; ++j) {
      sm[wave * G + j] = m[j];
      sl[wave * G + j] = l[j];
    }
  }
  if (has_d) {
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

// ------------------------------------------------------- MFMA form --
// For head dims 64 / 128 and 2..16 query heads per KV head, with 16-byte
// aligned rows.  A workgroup owns one KV head and a tile of 16 query rows
// (16 / G tokens x the G heads of the group) and all keys; its 8 wavefronts
// take interleaved 32-key chunks.  Per chunk a wavefront computes the
// 16 x 32 score tile with v_mfma_f32_16x16x32_bf16 (A = query rows, B = key
// rows: both 8 consecutive head-dim elements per lane, straight from
// memory), applies the scale and the mask, updates its online softmax per
// row (rows 4 (l / 16) + i of lane l, reduced over the 16 lanes that share
// them), and adds P.V with P (bf16) read back from LDS as the A operand and
// the chunk's value rows staged in LDS (B: 8 keys of one head-dim column per
// lane).  The 8 wavefront states are merged in wavefront order, so the
// result is run-to-run identical.
constexpr int kMfmaWaves = 8;
constexpr int kKeysPerChunk = 32;
constexpr int kPRow = kKeysPerChunk * 2 + 16;  // P row in LDS (bytes, padded)

template <int D>
constexpr int v_row_bytes() { return D * 2 + 8; }  // 8 B pad: the four 8-row groups hit distinct banks

template <int D>
constexpr size_t mfma_lds_bytes() {
  constexpr size_t loop = kMfmaWaves * (kKeysPerChunk * v_row_bytes<D>() + 16 * kPRow);
  constexpr size_t merge = kMfmaWaves * 16 * (D + 2) * sizeof(float);
  return loop > merge ? loop : merge;
}

__device__ __forceinline__ sf_f32x4 mfma_bf16(uint4 a, uint4 b, sf_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sf_bf16x8, a),
                                                 __builtin_bit_cast(sf_bf16x8, b), c, 0, 0, 0);
}

// Max / sum over the 16 lanes of a lane's row group (lanes 16 g .. 16 g + 15,
// one DPP row): the group_sum moves, with max for the max.
template <int CTRL>
__device__ __forceinline__ float dpp_max(float x) {
  const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false);
  return fmaxf(x, __int_as_float(moved));
}

__device__ __forceinline__ float row16_max(float x) {
  x = dpp_max<0xB1>(x);
  x = dpp_max<0x4E>(x);
  x = dpp_max<0x141>(x);
  return dpp_max<0x140>(x);
}

__device__ __forceinline__ float row16_sum(float x) { return group_sum<16>(x); }

template <int G, int D>
__global__ __launch_bounds__(kMfmaWaves * SF_WAVE) void tree_attention_mfma_kernel(
    const AttnArgs a) {
  constexpr int kTok = 16 / G;        // tokens per 16-row tile
  constexpr int kSteps = D / 32;      // MFMA k-steps of a score tile
  constexpr int kNt = D / 16;         // 16-wide head-dim tiles of the output
  constexpr int kVRow = v_row_bytes<D>();
  __shared__ __attribute__((aligned(16))) char lds[mfma_lds_bytes<D>()];
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int g4 = lane >> 4;           // row group of the C layout / k group of A, B
  const int col = lane & 15;
  const int h = blockIdx.x % a.Hkv;
  const int t0 = (blockIdx.x / a.Hkv) * kTok;
  char* vtile = lds + wave * kKeysPerChunk * kVRow;                       // [32][D] bf16
  char* ptile = lds + kMfmaWaves * kKeysPerChunk * kVRow + wave * 16 * kPRow;  // [16][32] bf16

  // A operand: query row `col` of the tile (token t0 + col / G, head h G + col % G).
  uint4 qa[kSteps];
  {
    const int t = min(t0 + col / G, a.Q - 1);
    const uint16_t* qr = a.q + t * a.q_tok + static_cast<int64_t>(h * G + col % G) * a.q_head;
#pragma unroll
    for (int s = 0; s < kSteps; ++s)
      qa[s] = *reinterpret_cast<const uint4*>(qr + 32 * s + 8 * g4);
  }
  // Rows of this lane in the C layout: 4 g4 + i, token t0 + (4 g4 + i) / G.
  int tok[4];
  bool row_ok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    tok[i] = t0 + (4 * g4 + i) / G;
    row_ok[i] = tok[i] < a.Q;
  }
  const uint16_t* kh = a.k + h * a.k_head;
  const uint16_t* vh = a.v + h * a.v_head;
  float m[4], l[4];
  sf_f32x4 acc[kNt];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
  }
#pragma unroll
  for (int nt = 0; nt < kNt; ++nt) acc[nt] = sf_f32x4{0.f, 0.f, 0.f, 0.f};

  // Chunk loads (keys, value rows, mask bits) are issued one chunk ahead.
  constexpr int kLanesPerRow = D / 8;
  constexpr int kRowsPerLoad = SF_WAVE / kLanesPerRow;
  constexpr int kVLoads = kKeysPerChunk / kRowsPerLoad;
  constexpr int kStride = kMfmaWaves * kKeysPerChunk;
  uint4 kf[2][kSteps], vv[kVLoads];
  uint32_t okbits = 0;  // bit 4 ct + i: key kb + 16 ct + col admitted for row 4 g4 + i
  auto load_chunk = [&](int kb) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      // Key fragments (B): key kb + 16 ct + col, head-dim 32 s + 8 g4.
      const uint16_t* kr = kh + min(kb + 16 * ct + col, a.S - 1) * a.k_tok + 8 * g4;
#pragma unroll
      for (int s = 0; s < kSteps; ++s) kf[ct][s] = *reinterpret_cast<const uint4*>(kr + 32 * s);
    }
    // Value rows kb .. kb + 31 (rows past the end repeat the last key: finite
    // values that meet p = 0).
#pragma unroll
    for (int j = 0; j < kVLoads; ++j) {
      const int r = j * kRowsPerLoad + lane / kLanesPerRow;
      vv[j] = *reinterpret_cast<const uint4*>(vh + min(kb + r, a.S - 1) * a.v_tok +
                                              8 * (lane % kLanesPerRow));
    }
    okbits = 0;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int key = kb + 16 * ct + col;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // Rows of one token share its mask byte (consecutive rows 4 g4 + i).
        bool ok = row_ok[i] && key < a.S;
        if (ok) ok = a.mask ? a.mask[tok[i] * a.mask_q + key] != 0 : key <= a.S - a.Q + tok[i];
        okbits |= static_cast<uint32_t>(ok) << (4 * ct + i);
      }
    }
  };
  if (wave * kKeysPerChunk < a.S) load_chunk(wave * kKeysPerChunk);
  for (int kb = wave * kKeysPerChunk; kb < a.S; kb += kStride) {
    uint4 kc[2][kSteps];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int s = 0; s < kSteps; ++s) kc[ct][s] = kf[ct][s];
    const uint32_t okc = okbits;
    // The chunk's value rows into this wavefront's LDS tile.
#pragma unroll
    for (int j = 0; j < kVLoads; ++j) {
      const int r = j * kRowsPerLoad + lane / kLanesPerRow;
      uint2* dst = reinterpret_cast<uint2*>(vtile + r * kVRow + 16 * (lane % kLanesPerRow));
      dst[0] = make_uint2(vv[j].x, vv[j].y);
      dst[1] = make_uint2(vv[j].z, vv[j].w);
    }
    if (kb + kStride < a.S) load_chunk(kb + kStride);
    // Scores of the 16 x 32 tile.
    sf_f32x4 sc[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      sc[ct] = sf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kSteps; ++s) sc[ct] = mfma_bf16(qa[s], kc[ct][s], sc[ct]);
    }
    // Online softmax per row.
    float p[2][4];
    float alpha[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bool ok[2];
      float x[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        ok[ct] = (okc >> (4 * ct + i)) & 1u;
        x[ct] = sc[ct][i] * a.scale;
      }
      const float cmax = row16_max(fmaxf(ok[0] ? x[0] : -INFINITY, ok[1] ? x[1] : -INFINITY));
      const float mnew = fmaxf(m[i], cmax);
      alpha[i] = 1.f;
      p[0][i] = p[1][i] = 0.f;
      if (mnew != -INFINITY) {
        alpha[i] = m[i] == -INFINITY ? 0.f : __expf(m[i] - mnew);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
          if (ok[ct]) p[ct][i] = __expf(x[ct] - mnew);
      }
      l[i] = l[i] * alpha[i] + row16_sum(p[0][i] + p[1][i]);
      m[i] = mnew;
    }
#pragma unroll
    for (int nt = 0; nt < kNt; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[nt][i] *= alpha[i];
    // P (bf16) through LDS into the A layout: row col, keys 8 g4 .. 8 g4 + 7.
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<uint16_t*>(ptile + (4 * g4 + i) * kPRow + 2 * (16 * ct + col)) =
            sf_f32_to_bf16(p[ct][i]);
    // The V and P tiles are this wavefront's own: its LDS accesses run in
    // order, and the fence keeps the compiler from moving the reads above.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const uint4 pa = *reinterpret_cast<const uint4*>(ptile + col * kPRow + 16 * g4);
    // P.V: B = value rows 8 g4 .. 8 g4 + 7 of head-dim column 16 nt + col.
#pragma unroll
    for (int nt = 0; nt < kNt; ++nt) {
      uint32_t w[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const char* v0 = vtile + (8 * g4 + 2 * jj) * kVRow + 2 * (16 * nt + col);
        const uint32_t lo = *reinterpret_cast<const uint16_t*>(v0);
        const uint32_t hi = *reinterpret_cast<const uint16_t*>(v0 + kVRow);
        w[jj] = lo | (hi << 16);
      }
      acc[nt] = mfma_bf16(pa, make_uint4(w[0], w[1], w[2], w[3]), acc[nt]);
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // tiles reused by the next chunk
  }

  // Merge the wavefront states in wavefront order.  The merge state overlays
  // the tiles of every wavefront: all of them have left the chunk loop first.
  __syncthreads();
  float* mst = reinterpret_cast<float*>(lds);                        // [waves][16] max
  float* lst = mst + kMfmaWaves * 16;                                 // [waves][16] sum
  float* ast = lst + kMfmaWaves * 16;                                 // [waves][16][D] acc
  if (col == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mst[wave * 16 + 4 * g4 + i] = m[i];
      lst[wave * 16 + 4 * g4 + i] = l[i];
    }
  }
#pragma unroll
  for (int nt = 0; nt < kNt; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) ast[(wave * 16 + 4 * g4 + i) * D + 16 * nt + col] = acc[nt][i];
  __syncthreads();
  const int Hq = a.Hkv * G;
  for (int o = threadIdx.x; o < 16 * D; o += kMfmaWaves * SF_WAVE) {
    const int r = o / D;
    const int d = o - r * D;
    const int t = t0 + r / G;
    if (t >= a.Q) continue;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kMfmaWaves; ++w) M = fmaxf(M, mst[w * 16 + r]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kMfmaWaves; ++w) {
        const float mw = mst[w * 16 + r];
        if (mw == -INFINITY) continue;
        const float f = __expf(mw - M);
        L = __builtin_fmaf(lst[w * 16 + r], f, L);
        O = __builtin_fmaf(ast[(w * 16 + r) * D + d], f, O);
      }
    }
    const float out = L > 0.f ? O / L : 0.f;
    a.out[(static_cast<int64_t>(t) * Hq + h * G + r % G) * D + d] = sf_f32_to_bf16(out);
  }
}

template <int G, int D>
int launch_mfma(const AttnArgs& a, hipStream_t s) {
  constexpr int kTok = 16 / G;
  const dim3 grid(static_cast<unsigned>((a.Q + kTok - 1) / kTok) * a.Hkv);
  tree_attention_mfma_kernel<G, D><<<grid, dim3(kMfmaWaves * SF_WAVE), 0, s>>>(a);
  SF_LAUNCH_CHECK();
  return SF_OK;
}

// Wavefronts per workgroup: 8 up to 8 heads per group, 4 for 16 (LDS).
constexpr int waves_for(int G) { return G <= 8 ? 8 : 4; }

// LDS bytes of one workgroup: query rows, merge state, and the larger of
// the chunk probabilities and the merge accumulators.
size_t lds_bytes(int G, int D) {
  const size_t w = waves_for(G);
  const size_t shared = w * G * (D > kChunk ? D : kChunk);
  return sizeof(float) * (static_cast<size_t>(G) * D + 2 * w * G + shared);
}

constexpr size_t kMaxLds = 64 * 1024;

template <int G>
int launch_g(const AttnArgs& a, hipStream_t s) {
  constexpr int NW = waves_for(G);
  const size_t lds = lds_bytes(G, a.D);
  const dim3 grid(static_cast<unsigned>(a.Q) * a.Hkv);
  const dim3 block(NW * SF_WAVE);
  // Fixed head dims 64 / 128 up to 8 heads per group (more would spill).
  if (G <= 8 && a.D == 128)
    tree_attention_kernel<G, (G <= 8 ? 16 : 0), 2, NW><<<grid, block, lds, s>>>(a);
  else if (G <= 8 && a.D == 64)
    tree_attention_kernel<G, (G <= 8 ? 8 : 0), 1, NW><<<grid, block, lds, s>>>(a);
  else if (a.D <= SF_WAVE)
    tree_attention_kernel<G, 0, 1, NW><<<grid, block, lds, s>>>(a);
  else if (a.D <= 2 * SF_WAVE)
    tree_attention_kernel<G, 0, 2, NW><<<grid, block, lds, s>>>(a);
  else
    tree_attention_kernel<G, 0, 4, NW><<<grid, block, lds, s>>>(a);
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
  // The MFMA form: 16-byte aligned query / key / value rows (8-element
  // strides), head dim 64 or 128, 2..16 query heads per KV head.
  const bool rows16 = aligned(q, 16) && aligned(k, 16) && aligned(v, 16) &&
                      q_stride_token % 8 == 0 && q_stride_head % 8 == 0 &&
                      v_stride_token % 8 == 0 && v_stride_head % 8 == 0;
  if (rows16 && head_dim == 128) {
    switch (G) {
      case 2: return launch_mfma<2, 128>(a, s);
      case 4: return launch_mfma<4, 128>(a, s);
      case 8: return launch_mfma<8, 128>(a, s);
      case 16: return launch_mfma<16, 128>(a, s);
      default: break;
    }
  } else if (rows16 && head_dim == 64) {
    switch (G) {
      case 2: return launch_mfma<2, 64>(a, s);
      case 4: return launch_mfma<4, 64>(a, s);
      case 8: return launch_mfma<8, 64>(a, s);
      case 16: return launch_mfma<16, 64>(a, s);
      default: break;
    }
  }
  switch (G) {
    case 1: return launch_g<1>(a, s);
    case 2: return launch_g<2>(a, s);
    case 4: return launch_g<4>(a, s);
    case 8: return launch_g<8>(a, s);
    case 16: return launch_g<16>(a, s);
    default: return SF_ERR_UNSUPPORTED_SHAPE;
  }
}
