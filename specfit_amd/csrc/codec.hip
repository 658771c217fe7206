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
//            list (so a workgroup finds its escapes with two loads).
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

__global__ __launch_bounds__(kThreads) void decode_kernel(const DecodeArgs a) {
  __shared__ uint8_t table[16];
  if (threadIdx.x < 16)
    table[threadIdx.x] = static_cast<uint8_t>(a.table[threadIdx.x >> 2] >> (8 * (threadIdx.x & 3)));
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kChunk;
  const int64_t c1 = c0 + kChunk < a.n ? c0 + kChunk : a.n;
  __syncthreads();
  const int64_t i = c0 + static_cast<int64_t>(threadIdx.x) * kPerThread;
  if (i + kPerThread <= a.n) {
    const uint4 s = *reinterpret_cast<const uint4*>(a.sm + i);
    const uint2 x = *reinterpret_cast<const uint2*>(a.codes + (i >> 1));
    const uint32_t sw[4] = {s.x, s.y, s.z, s.w};
    const uint32_t xw[2] = {x.x, x.y};
    uint32_t w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      // values 2k and 2k+1 of the thread: bytes 2k, 2k+1 of S, byte k of X
      const uint32_t sm0 = (sw[k >> 1] >> (16 * (k & 1))) & 0xffu;
      const uint32_t sm1 = (sw[k >> 1] >> (16 * (k & 1) + 8)) & 0xffu;
      const uint32_t xb = (xw[k >> 2] >> (8 * (k & 3))) & 0xffu;
      w[k] = join(sm0, table[xb & 15u]) | (join(sm1, table[xb >> 4]) << 16);
    }
    uint4* o = reinterpret_cast<uint4*>(a.out + i);
    o[0] = make_uint4(w[0], w[1], w[2], w[3]);
    o[1] = make_uint4(w[4], w[5], w[6], w[7]);
  } else {
    for (int64_t j = i; j < a.n && j < i + kPerThread; ++j) {
      const uint32_t xb = a.codes[j >> 1];
      const uint32_t code = (j & 1) ? xb >> 4 : xb & 15u;
      a.out[j] = static_cast<uint16_t>(join(a.sm[j], table[code]));
    }
  }
  if (a.n_esc > 0) {
    // The chunk's escapes, clamped to the list (a malformed table only
    // skips or repeats patches inside the chunk, never writes outside it).
    const int first = min(static_cast<int>(a.chunk_esc[blockIdx.x]), a.n_esc);
    const int last = min(static_cast<int>(a.chunk_esc[blockIdx.x + 1]), a.n_esc);
    __syncthreads();  // the chunk's plain values are written
    for (int e = first + static_cast<int>(threadIdx.x); e < last; e += kThreads) {
      const int64_t j = a.esc_idx[e];
      if (j >= c0 && j < c1) a.out[j] = static_cast<uint16_t>(join(a.sm[j], a.esc_exp[e]));
    }
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
