// Expert-weight decoder for the host-to-device path (gfx950).
//
// An expert moves over the host link as an exponent-coded record of its bf16
// weights instead of the raw 2 bytes per value.  A bf16 value is
// sign (1 bit) | exponent (8 bits) | mantissa (7 bits).  Weights of a layer
// span only a few dozen binades, most of them a dozen, so the record stores
//   plane S: one byte per value, sign << 7 | mantissa;
//   plane X: one 4-bit code per value (value 2j in the low nibble of byte j):
//            code c < 15 stands for exponent table[c], code 15 for an escape;
//   escapes: the index (uint32, ascending) and exponent byte of every value
//            whose exponent is not in the table, and for every chunk of
//            SF_DECODE_CHUNK values the position of its first escape in that
//            list.  The decode reads only the exponents: an escape's position
//            in the list is the chunk's first plus its rank in the chunk.
// 12 bits per value plus the escapes: 75% of the raw bytes for experts whose
// values fit 15 exponents.  The decode restores every value's 16 bits
// exactly (no rounding anywhere), so a decoded slot holds the same bytes as
// a raw copy.
//
// Record layout (byte offsets, every section 256-byte aligned):
//   S at 0 (n bytes), X at align(n), escape indices at
//   align(n) + align(ceil(n / 2)), escape exponents after them at
//   + align(4 * escapes), the chunk table (ceil(n / SF_DECODE_CHUNK) + 1
//   uint32) after those at + align(escapes).
#include "sf_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 16;                           // values per thread
constexpr int64_t kChunk = int64_t{kThreads} * kPerThread;  // values per workgroup
static_assert(kChunk == SF_DECODE_CHUNK, "a workgroup decodes one chunk of the record");

int64_t align256(int64_t x) { return (x + 255) & ~int64_t{255}; }

struct DecodeArgs {
  const uint8_t* sm;        // plane S
  const uint8_t* codes;     // plane X
  const uint32_t* esc_idx;  // escape indices, ascending
  const uint8_t* esc_exp;   // escape exponents
  const uint32_t* chunk_esc;  // first escape of each chunk, [chunks + 1]
  uint16_t* out;            // bf16 [n]
  int64_t n;
  int n_esc;
  uint32_t table[4];        // exponent table, byte c = exponent of code c
};

__device__ __forceinline__ uint32_t join(uint32_t sm, uint32_t exponent) {
  return ((sm & 0x80u) << 8) | (exponent << 7) | (sm & 0x7fu);
}

// Exclusive prefix over the wavefront of v (0 <= v <= 16) and the wavefront
// total, from one ballot per bit of v.
__device__ __forceinline__ int wave_prefix(int v, int& total) {
  int prefix = 0;
  total = 0;
#pragma unroll
  for (int b = 0; b < 5; ++b) {
    const uint64_t m = __ballot((v >> b) & 1);
    const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
    prefix += below << b;
    total += __popcll(m) << b;
  }
  return prefix;
}

// One workgroup per chunk; thread t decodes values c0 + 16 t .. + 15.  An
// escaped value (code 15) takes the exponent at its rank among the chunk's
// escapes (value order), counted from the chunk's first escape; the ranks
// come from a workgroup prefix over per-thread escape counts, so every value
// is written once and only escapes read the escape list.
__global__ __launch_bounds__(kThreads) void decode_kernel(const DecodeArgs a) {
  __shared__ uint8_t table[16];
  __shared__ int wave_total[kThreads / SF_WAVE];
  const int tid = threadIdx.x;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kChunk;
  const int64_t i = c0 + static_cast<int64_t>(tid) * kPerThread;
  const int nv = i >= a.n ? 0 : (a.n - i < kPerThread ? static_cast<int>(a.n - i) : kPerThread);
  uint32_t sw[4] = {0, 0, 0, 0};
  uint32_t xw[2] = {0, 0};
  if (nv == kPerThread) {
    const uint4 s = *reinterpret_cast<const uint4*>(a.sm + i);
    const uint2 x = *reinterpret_cast<const uint2*>(a.codes + (i >> 1));
    sw[0] = s.x; sw[1] = s.y; sw[2] = s.z; sw[3] = s.w;
    xw[0] = x.x; xw[1] = x.y;
  } else {
    // Tail of the record: values past n keep code 0 (never an escape).
    for (int k = 0; k < nv; ++k) {
      sw[k >> 2] |= static_cast<uint32_t>(a.sm[i + k]) << (8 * (k & 3));
      const uint32_t xb = a.codes[(i + k) >> 1];
      const uint32_t code = ((i + k) & 1) ? xb >> 4 : xb & 15u;
      xw[k >> 3] |= code << (4 * (k & 7));
    }
  }
  // The chunk's escapes: list positions [first, last) (clamped to the list,
  // so a malformed table cannot read past it).
  int first = 0, last = 0;
  if (a.n_esc > 0) {
    first = min(static_cast<int>(a.chunk_esc[blockIdx.x]), a.n_esc);
    last = min(static_cast<int>(a.chunk_esc[blockIdx.x + 1]), a.n_esc);
  }
  if (tid < 16)
    table[tid] = static_cast<uint8_t>(a.table[tid >> 2] >> (8 * (tid & 3)));
  // 4-bit codes of the thread's values, and which are escapes.
  uint32_t esc_mask = 0;
#pragma unroll
  for (int k = 0; k < kPerThread; ++k)
    if (((xw[k >> 3] >> (4 * (k & 7))) & 15u) == 15u) esc_mask |= 1u << k;
  int rank = first;
  if (last > first) {  // uniform: the chunk has escapes
    int total;
    rank += wave_prefix(__popc(esc_mask), total);
    if ((tid & (SF_WAVE - 1)) == 0) wave_total[tid / SF_WAVE] = total;
  }
  __syncthreads();  // the table (and the wavefront totals)
  if (last > first) {
    for (int w = 0; w < tid / SF_WAVE; ++w) rank += wave_total[w];
  }
  uint32_t w16[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t sm0 = (sw[k >> 1] >> (16 * (k & 1))) & 0xffu;
    const uint32_t sm1 = (sw[k >> 1] >> (16 * (k & 1) + 8)) & 0xffu;
    const uint32_t xb = (xw[k >> 2] >> (8 * (k & 3))) & 0xffu;
    w16[k] = join(sm0, table[xb & 15u]) | (join(sm1, table[xb >> 4]) << 16);
  }
  // Escapes of this thread, in value order (rare: a few per expert chunk).
  for (uint32_t m = esc_mask; m; m &= m - 1) {
    const int k = __builtin_ctz(m);
    if (rank < last) {
      const uint32_t sm = (sw[k >> 2] >> (8 * (k & 3))) & 0xffu;
      const uint32_t v = join(sm, a.esc_exp[rank]);
      const int h = 16 * (k & 1);
      w16[k >> 1] = (w16[k >> 1] & ~(0xffffu << h)) | (v << h);
    }
    ++rank;
  }
  if (nv == kPerThread) {
    uint4* o = reinterpret_cast<uint4*>(a.out + i);
    o[0] = make_uint4(w16[0], w16[1], w16[2], w16[3]);
    o[1] = make_uint4(w16[4], w16[5], w16[6], w16[7]);
  } else {
    for (int k = 0; k < nv; ++k)
      a.out[i + k] = static_cast<uint16_t>(w16[k >> 1] >> (16 * (k & 1)));
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int64_t chunk_table_offset(int64_t n_values, int64_t n_escapes) {
  return align256(n_values) + align256((n_values + 1) / 2) + align256(4 * n_escapes) +
         align256(n_escapes);
}

}  // namespace

extern "C" int64_t sf_expert_record_bytes(int64_t n_values, int64_t n_escapes) {
  if (n_values < 0 || n_escapes < 0 || n_escapes > n_values) return -1;
  const int64_t chunks = (n_values + kChunk - 1) / kChunk;
  return chunk_table_offset(n_values, n_escapes) + align256(4 * (chunks + 1));
}

extern "C" int sf_expert_decode(const void* record, size_t record_bytes, int64_t n_values,
                                const uint8_t* exponent_table, int n_escapes, void* out,
                                sf_stream_t stream) {
  if (n_values < 0 || n_escapes < 0 || n_escapes > n_values || n_values > 0xffffffffLL)
    return SF_ERR_INVALID_ARGUMENT;
  if (n_values == 0) return SF_OK;
  if (!record || !exponent_table || !out) return SF_ERR_INVALID_ARGUMENT;
  if (static_cast<int64_t>(record_bytes) < sf_expert_record_bytes(n_values, n_escapes))
    return SF_ERR_INVALID_ARGUMENT;
  if (!aligned16(record) || !aligned16(out)) return SF_ERR_MISALIGNED;
  const uint8_t* base = static_cast<const uint8_t*>(record);
  DecodeArgs a{};
  a.sm = base;
  a.codes = base + align256(n_values);
  a.esc_idx = reinterpret_cast<const uint32_t*>(a.codes + align256((n_values + 1) / 2));
  a.esc_exp = reinterpret_cast<const uint8_t*>(a.esc_idx) + align256(4 * int64_t{n_escapes});
  a.chunk_esc = reinterpret_cast<const uint32_t*>(base + chunk_table_offset(n_values, n_escapes));
  a.out = static_cast<uint16_t*>(out);
  a.n = n_values;
  a.n_esc = n_escapes;
  for (int c = 0; c < 16; ++c)
    a.table[c >> 2] |= static_cast<uint32_t>(exponent_table[c]) << (8 * (c & 3));
  const int64_t blocks = (n_values + kChunk - 1) / kChunk;
  decode_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                  reinterpret_cast<hipStream_t>(stream)>>>(a);
  SF_LAUNCH_CHECK();
  return SF_OK;
}
