// Expert-weight decoder for the host-to-device path (gfx950).
//
// An expert moves over the host link as an exponent-coded record of its bf16
// weights instead of the raw 2 bytes per value.  A bf16 value is
// sign (1 bit) | exponent (8 bits) | mantissa (7 bits), and the weights of
// an expert concentrate their exponents in a few binades.  The record:
//   S   one byte per value, sign << 7 | mantissa;
//   P   a 3-bit primary code per value, as three bit planes (plane p holds
//       bit p of the codes of values 16g .. 16g+15 in its uint16 word g):
//       code c < 7 stands for exponent primary[c], code 7 for "secondary";
//   Q   one 4-bit secondary code per value with primary code 7, in value
//       order (entry 2j in the low nibble of byte j): code c < 15 stands for
//       exponent secondary[c], code 15 for "raw";
//   R   the exponent byte of every value with secondary code 15, in value
//       order;
//   QC, RC  per chunk of SF_DECODE_CHUNK values, the number of Q and R
//       entries of the values before it (chunks + 1 uint32 each).
// About 11.1 bits per value for N(0, 0.02) weights (98% of values in 7
// binades, all but a few values per expert in 22): 69% of the raw bytes.  The decode restores
// every value's 16 bits exactly, so a decoded slot holds the same bytes as a
// raw copy.
//
// Record layout (byte offsets, every section 256-byte aligned), for n
// values, q secondary and r raw entries:
//   S at 0 [n], P at align(n) [3 planes of 2 * ceil(n / 16) bytes, each
//   aligned], Q [ceil(q / 2)], R [r], QC [4 (chunks + 1)], RC [4 (chunks + 1)].
#include "sf_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 16;                           // values per thread
constexpr int64_t kChunk = int64_t{kThreads} * kPerThread;  // values per workgroup
static_assert(kChunk == SF_DECODE_CHUNK, "a workgroup decodes one chunk of the record");
constexpr int kWaves = kThreads / SF_WAVE;

int64_t align256(int64_t x) { return (x + 255) & ~int64_t{255}; }

struct Layout {
  int64_t plane, q, r, qc, rc, total;  // byte offsets of P plane 0, Q, R, QC, RC; size
};

Layout layout(int64_t n, int64_t q, int64_t r) {
  Layout l;
  const int64_t chunks = (n + kChunk - 1) / kChunk;
  const int64_t plane_bytes = align256(2 * ((n + 15) / 16));
  l.plane = align256(n);
  l.q = l.plane + 3 * plane_bytes;
  l.r = l.q + align256((q + 1) / 2);
  l.qc = l.r + align256(r);
  l.rc = l.qc + align256(4 * (chunks + 1));
  l.total = l.rc + align256(4 * (chunks + 1));
  return l;
}

struct DecodeArgs {
  const uint8_t* sm;       // S
  const uint16_t* planes;  // P plane 0; plane p at planes + p * plane_words
  int64_t plane_words;
  const uint8_t* sec;      // Q
  const uint8_t* raw;      // R
  const uint32_t* q_chunk; // QC
  const uint32_t* r_chunk; // RC
  uint16_t* out;           // bf16 [n]
  int64_t n;
  int n_sec;
  int n_raw;
  uint32_t table[8];       // bytes 0..7: primary exponents; 16..31: secondary
};

__device__ __forceinline__ uint32_t join(uint32_t sm, uint32_t exponent) {
  return ((sm & 0x80u) << 8) | (exponent << 7) | (sm & 0x7fu);
}

// Exclusive prefix over the workgroup of v (0 <= v <= 16) in thread order,
// from one ballot per bit of v and the wavefront totals in LDS.  Every
// thread of the workgroup calls it (it holds a barrier).
__device__ __forceinline__ int workgroup_prefix(int v, int* wave_total) {
  int prefix = 0, total = 0;
#pragma unroll
  for (int b = 0; b < 5; ++b) {
    const uint64_t m = __ballot((v >> b) & 1);
    prefix += __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0))
              << b;
    total += __popcll(m) << b;
  }
  const int wave = threadIdx.x / SF_WAVE;
  if ((threadIdx.x & (SF_WAVE - 1)) == 0) wave_total[wave] = total;
  __syncthreads();
  for (int w = 0; w < wave; ++w) prefix += wave_total[w];
  return prefix;
}

// One workgroup per chunk; thread t decodes values c0 + 16 t .. + 15.  A
// value with primary code 7 takes the secondary code at its rank among the
// chunk's primary escapes (value order) from the chunk's first Q entry; one
// with secondary code 15 takes the raw exponent at its rank among the
// chunk's raw entries.  Ranks come from workgroup prefixes over per-thread
// counts, so every value is written once.
__global__ __launch_bounds__(kThreads) void decode_kernel(const DecodeArgs a) {
  __shared__ uint8_t table[32];
  __shared__ int wave_total[2][kWaves];
  const int tid = threadIdx.x;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kChunk;
  const int64_t i = c0 + static_cast<int64_t>(tid) * kPerThread;
  const int nv = i >= a.n ? 0 : (a.n - i < kPerThread ? static_cast<int>(a.n - i) : kPerThread);
  const int64_t g = i / kPerThread;  // the thread's word in each plane
  uint32_t sw[4] = {0, 0, 0, 0};
  uint32_t p0 = 0, p1 = 0, p2 = 0;
  if (nv > 0) {
    // Plane words exist for every group, a partial last one included (its
    // bits past n are 0).
    p0 = a.planes[g];
    p1 = a.planes[a.plane_words + g];
    p2 = a.planes[2 * a.plane_words + g];
  }
  if (nv == kPerThread) {
    const uint4 s = *reinterpret_cast<const uint4*>(a.sm + i);
    sw[0] = s.x; sw[1] = s.y; sw[2] = s.z; sw[3] = s.w;
  } else {
    for (int k = 0; k < nv; ++k) sw[k >> 2] |= static_cast<uint32_t>(a.sm[i + k]) << (8 * (k & 3));
  }
  // The chunk's Q and R ranges, clamped to the lists (a malformed table can
  // only skip or repeat entries, never read past a list).
  int q_first = 0, q_last = 0, r_first = 0, r_last = 0;
  if (a.n_sec > 0) {
    q_first = min(static_cast<int>(a.q_chunk[blockIdx.x]), a.n_sec);
    q_last = min(static_cast<int>(a.q_chunk[blockIdx.x + 1]), a.n_sec);
  }
  if (a.n_raw > 0) {
    r_first = min(static_cast<int>(a.r_chunk[blockIdx.x]), a.n_raw);
    r_last = min(static_cast<int>(a.r_chunk[blockIdx.x + 1]), a.n_raw);
  }
  if (tid < 32) table[tid] = static_cast<uint8_t>(a.table[tid >> 2] >> (8 * (tid & 3)));
  // Primary codes (bit j of p0 | p1 << 1 | p2 << 2); code 7 is an escape.
  const uint32_t esc1 = p0 & p1 & p2;
  int q_rank = q_first;
  if (q_last > q_first) q_rank += workgroup_prefix(__popc(esc1), wave_total[0]);
  __syncthreads();  // the tables
  uint32_t w16[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    uint32_t v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = 2 * k + h;
      const uint32_t c = ((p0 >> j) & 1u) | (((p1 >> j) & 1u) << 1) | (((p2 >> j) & 1u) << 2);
      v[h] = join((sw[j >> 2] >> (8 * (j & 3))) & 0xffu, table[c]);
    }
    w16[k] = v[0] | (v[1] << 16);
  }
  // Secondary codes of this thread's escapes, in value order, packed four
  // bits per value; the raw ones among them are counted for their ranks.
  uint64_t sec_codes = 0;
  uint32_t raw_mask = 0;
  for (uint32_t m = esc1; m; m &= m - 1) {
    const int k = __builtin_ctz(m);
    uint32_t c = 15;
    if (q_rank < q_last) {
      const uint32_t byte = a.sec[q_rank >> 1];
      c = (q_rank & 1) ? byte >> 4 : byte & 15u;
    }
    sec_codes |= static_cast<uint64_t>(c) << (4 * k);
    if (c == 15) raw_mask |= 1u << k;
    ++q_rank;
  }
  int r_rank = r_first;
  if (r_last > r_first) r_rank += workgroup_prefix(__popc(raw_mask), wave_total[1]);
  for (uint32_t m = esc1; m; m &= m - 1) {
    const int k = __builtin_ctz(m);
    uint32_t e;
    if (raw_mask & (1u << k)) {
      if (r_rank >= r_last) continue;  // malformed record: leave the value
      e = a.raw[r_rank++];
    } else {
      e = table[16 + ((sec_codes >> (4 * k)) & 15u)];
    }
    const uint32_t v = join((sw[k >> 2] >> (8 * (k & 3))) & 0xffu, e);
    const int h = 16 * (k & 1);
    w16[k >> 1] = (w16[k >> 1] & ~(0xffffu << h)) | (v << h);
  }
  if (nv == kPerThread) {
    uint4* o = reinterpret_cast<uint4*>(a.out + i);
    o[0] = make_uint4(w16[0], w16[1], w16[2], w16[3]);
    o[1] = make_uint4(w16[4], w16[5], w16[6], w16[7]);
  } else {
    for (int k = 0; k < nv; ++k) a.out[i + k] = static_cast<uint16_t>(w16[k >> 1] >> (16 * (k & 1)));
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool counts_valid(int64_t n, int64_t q, int64_t r) {
  return n >= 0 && q >= 0 && r >= 0 && q <= n && r <= q;
}

}  // namespace

extern "C" int64_t sf_expert_record_bytes(int64_t n_values, int64_t n_secondary,
                                          int64_t n_raw) {
  if (!counts_valid(n_values, n_secondary, n_raw)) return -1;
  return layout(n_values, n_secondary, n_raw).total;
}

extern "C" int sf_expert_decode(const void* record, size_t record_bytes, int64_t n_values,
                                const uint8_t* exponent_table, int n_secondary, int n_raw,
                                void* out, sf_stream_t stream) {
  if (!counts_valid(n_values, n_secondary, n_raw) || n_values > 0xffffffffLL)
    return SF_ERR_INVALID_ARGUMENT;
  if (n_values == 0) return SF_OK;
  if (!record || !exponent_table || !out) return SF_ERR_INVALID_ARGUMENT;
  const Layout l = layout(n_values, n_secondary, n_raw);
  if (static_cast<int64_t>(record_bytes) < l.total) return SF_ERR_INVALID_ARGUMENT;
  if (!aligned16(record) || !aligned16(out)) return SF_ERR_MISALIGNED;
  const uint8_t* base = static_cast<const uint8_t*>(record);
  DecodeArgs a{};
  a.sm = base;
  a.planes = reinterpret_cast<const uint16_t*>(base + l.plane);
  a.plane_words = align256(2 * ((n_values + 15) / 16)) / 2;
  a.sec = base + l.q;
  a.raw = base + l.r;
  a.q_chunk = reinterpret_cast<const uint32_t*>(base + l.qc);
  a.r_chunk = reinterpret_cast<const uint32_t*>(base + l.rc);
  a.out = static_cast<uint16_t*>(out);
  a.n = n_values;
  a.n_sec = n_secondary;
  a.n_raw = n_raw;
  for (int c = 0; c < 32; ++c)
    a.table[c >> 2] |= static_cast<uint32_t>(exponent_table[c]) << (8 * (c & 3));
  const int64_t blocks = (n_values + kChunk - 1) / kChunk;
  decode_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                  reinterpret_cast<hipStream_t>(stream)>>>(a);
  SF_LAUNCH_CHECK();
  return SF_OK;
}
