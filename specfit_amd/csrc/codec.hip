// Expert-weight decoder for the host-to-device path (gfx950).
//
// An expert moves over the host link as an exponent-coded record of its bf16
// weights instead of the raw 2 bytes per value.  A bf16 value is
// sign (1 bit) | exponent (8 bits) | mantissa (7 bits).  The sign and
// mantissa bits of weights are close to uniform and stay as they are; the
// exponents concentrate in a few binades and take a cascade of short codes,
// each level a fixed-width code into a small table of the expert's own whose
// last code defers to the next level:
//   level 1  2 bits, every value:              c < 3: table[c],      3: level 2
//   level 2  2 bits, values with level-1 3:    c < 3: table[8 + c],  3: level 3
//   level 3  4 bits, values with level-2 3:    c < 15: table[16 + c], 15: raw
//   raw      the exponent byte.
// The record:
//   S       one byte per value, sign << 7 | mantissa;
//   P       the level-1 codes as two bit planes (plane p holds bit p of the
//           codes of values 16g .. 16g+15 in its uint16 word g);
//   L2, L3  the level-2 and level-3 codes in value order, packed from bit 0
//           of byte 0 upwards (2 and 4 bits per entry);
//   R       the raw exponent bytes in value order;
//   C2, C3, CR  per chunk of SF_DECODE_CHUNK values, the L2, L3 and R
//           entries of the values before it (chunks + 1 uint32 each).
// About 10.7 bits per value for N(0, 0.02) weights (73% of values in 3
// binades, all but 4% in 6): 67% of the raw bytes.  The decode restores
// every value's 16 bits exactly, so a decoded slot holds the same bytes as a
// raw copy.
//
// Record layout (byte offsets, every section 256-byte aligned), for n
// values with n2, n3 and nr entries in L2, L3 and R:
//   S at 0 [n], P at align(n) [2 planes of 2 * ceil(n / 16) bytes, each
//   aligned], L2 [ceil(n2 / 4)], L3 [ceil(n3 / 2)], R [nr],
//   C2, C3, CR [4 (chunks + 1)] each.
#include "sf_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 16;                           // values per thread
constexpr int64_t kChunk = int64_t{kThreads} * kPerThread;  // values per workgroup
static_assert(kChunk == SF_DECODE_CHUNK, "a workgroup decodes one chunk of the record");
constexpr int kWaves = kThreads / SF_WAVE;

int64_t align256(int64_t x) { return (x + 255) & ~int64_t{255}; }

struct Layout {
  int64_t plane, l2, l3, r, c2, c3, cr, total;  // byte offsets of the sections; size
};

Layout layout(int64_t n, int64_t n2, int64_t n3, int64_t nr) {
  Layout l;
  const int64_t chunks = (n + kChunk - 1) / kChunk;
  const int64_t plane_bytes = align256(2 * ((n + 15) / 16));
  const int64_t table_bytes = align256(4 * (chunks + 1));
  l.plane = align256(n);
  l.l2 = l.plane + 2 * plane_bytes;
  l.l3 = l.l2 + align256((n2 + 3) / 4);
  l.r = l.l3 + align256((n3 + 1) / 2);
  l.c2 = l.r + align256(nr);
  l.c3 = l.c2 + table_bytes;
  l.cr = l.c3 + table_bytes;
  l.total = l.cr + table_bytes;
  return l;
}

struct DecodeArgs {
  const uint8_t* sm;        // S
  const uint16_t* planes;   // P plane 0; plane 1 at planes + plane_words
  int64_t plane_words;
  const uint32_t* l2;       // L2 as words (the section is 256-byte aligned)
  const uint32_t* l3;       // L3 as words
  const uint8_t* raw;       // R
  const uint32_t* c2;       // C2, C3, CR
  const uint32_t* c3;
  const uint32_t* cr;
  uint16_t* out;            // bf16 [n]
  int64_t n;
  int n2, n3, nr;
  uint32_t table[8];        // bytes 0..2: level 1; 8..10: level 2; 16..30: level 3
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

// Bits bit0 .. bit0 + nbits - 1 (nbits <= 64) of a packed list, bit j of
// the result = list bit bit0 + j.  Loads only the words that hold those
// bits, which lie inside the list's bytes.
__device__ __forceinline__ uint64_t read_bits(const uint32_t* w, int64_t bit0, int nbits) {
  if (nbits <= 0) return 0;
  const int64_t first = bit0 >> 5;
  const int64_t last = (bit0 + nbits - 1) >> 5;
  const int sh = static_cast<int>(bit0 & 31);
  uint64_t v = static_cast<uint64_t>(w[first]) >> sh;
  if (last > first) v |= static_cast<uint64_t>(w[first + 1]) << (32 - sh);
  if (last > first + 1) v |= static_cast<uint64_t>(w[first + 2]) << (64 - sh);  // sh > 0 here
  return nbits == 64 ? v : v & ((uint64_t{1} << nbits) - 1);
}

// Clamped entry range [first, last) of one list for chunk `chunk`: a
// malformed table can only skip or repeat entries, never read past a list.
__device__ __forceinline__ void chunk_range(const uint32_t* table, int count, int chunk,
                                            int& first, int& last) {
  first = last = 0;
  if (count > 0) {  // clamped as unsigned: an entry above INT_MAX is no negative rank
    first = static_cast<int>(min(table[chunk], static_cast<uint32_t>(count)));
    last = static_cast<int>(min(table[chunk + 1], static_cast<uint32_t>(count)));
  }
}

// Bit j of n (n < 16) moved to bit 8 j: the multiplier's four terms put bit j
// at j + 7 i, all distinct for i, j < 4, and only i = j lands on 8 j.
__device__ __forceinline__ uint32_t spread4(uint32_t n) {
  return __umul24(n, 0x00204081u) & 0x01010101u;
}

// Byte i of the result = byte sel_i of {hi (bytes 4..7) : lo (bytes 0..3)};
// selector byte 12 gives 0.
__device__ __forceinline__ uint32_t byte_perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// One workgroup per chunk; thread t decodes values 16 t .. 16 t + 15 of
// it.  A value that reaches level 2 or 3 takes the code at its rank among
// the chunk's values that reach that level, counted from the chunk's first
// entry of that level's list; a raw exponent likewise.  Ranks come from
// workgroup prefixes over per-thread counts (skipped for a list the chunk
// has no entries of), so every value is written once.  Entries a malformed
// record lacks count as the next level's escape; a value left without a raw
// byte keeps exponent 0.
//
// Exponents of levels 1 and 2 come four values at a time from one byte
// permute over table bytes 0..3 and 8..11: value j's selector is its level-1
// code, or 4 + its level-2 code when the level-1 code is 3 (selector 7, a
// level-3 value, is patched after).  Sign, exponent and mantissa bytes are
// joined four values at a time: the low byte of a bf16 value is its mantissa
// and exponent bit 0, the high byte its sign and exponent bits 1..7.
__global__ __launch_bounds__(kThreads) void decode_kernel(const DecodeArgs a) {
  __shared__ int wave_total[3][kWaves];
  const int tid = threadIdx.x;
  const int chunk = blockIdx.x;
  const int64_t i = static_cast<int64_t>(chunk) * kChunk + static_cast<int64_t>(tid) * kPerThread;
  const int nv = i >= a.n ? 0 : (a.n - i < kPerThread ? static_cast<int>(a.n - i) : kPerThread);
  const int64_t g = i / kPerThread;  // the thread's word in each plane
  uint32_t sw[4] = {0, 0, 0, 0};
  uint32_t p0 = 0, p1 = 0;
  if (nv > 0) {
    // Plane words exist for every group, a partial last one included (its
    // bits past n are 0).
    p0 = a.planes[g];
    p1 = a.planes[a.plane_words + g];
  }
  if (nv == kPerThread) {
    const uint4 s = *reinterpret_cast<const uint4*>(a.sm + i);
    sw[0] = s.x; sw[1] = s.y; sw[2] = s.z; sw[3] = s.w;
  } else {
    for (int k = 0; k < nv; ++k) sw[k >> 2] |= static_cast<uint32_t>(a.sm[i + k]) << (8 * (k & 3));
  }
  int f2, l2, f3, l3, fr, lr;
  chunk_range(a.c2, a.n2, chunk, f2, l2);
  chunk_range(a.c3, a.n3, chunk, f3, l3);
  chunk_range(a.cr, a.nr, chunk, fr, lr);

  // Level 2: this thread's entries are consecutive in L2 from rank r2.
  const uint32_t esc1 = p0 & p1;
  const int k1 = __popc(esc1);
  int r2 = f2;
  if (l2 > f2) r2 += workgroup_prefix(k1, wave_total[0]);
  const int v2 = max(0, min(k1, l2 - r2));
  uint32_t codes2 = static_cast<uint32_t>(read_bits(a.l2, 2 * static_cast<int64_t>(r2), 2 * v2));
  if (v2 < k1) codes2 |= ~0u << (2 * v2);  // missing entries escape
  // Bit j of c2lo / c2hi: bit 0 / bit 1 of value j's level-2 code (0 for a
  // value without one).
  uint32_t c2lo = 0, c2hi = 0;
  for (uint32_t m = esc1, c = codes2; m; m &= m - 1, c >>= 2) {
    const uint32_t bit = m & (0u - m);
    c2lo |= (c & 1u) ? bit : 0u;
    c2hi |= (c & 2u) ? bit : 0u;
  }
  const uint32_t esc2 = c2lo & c2hi;

  // Level 3: consecutive in L3 from rank r3.
  const int k2 = __popc(esc2);
  int r3 = f3;
  if (l3 > f3) r3 += workgroup_prefix(k2, wave_total[1]);
  const int v3 = max(0, min(k2, l3 - r3));
  uint64_t codes3 = read_bits(a.l3, 4 * static_cast<int64_t>(r3), 4 * v3);
  if (v3 < k2) codes3 |= ~uint64_t{0} << (4 * v3);
  uint32_t esc3 = 0;  // values with a raw exponent
  {
    uint64_t c = codes3;
    for (uint32_t m = esc2; m; m &= m - 1, c >>= 4)
      if ((static_cast<uint32_t>(c) & 15u) == 15u) esc3 |= m & (0u - m);
  }
  // Raw exponents: consecutive in R from rank rr.
  int rr = fr;
  if (lr > fr) rr += workgroup_prefix(__popc(esc3), wave_total[2]);

  uint32_t ew[4];  // exponent bytes of values 4w .. 4w+3
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t s1 = spread4((p0 >> (4 * w)) & 15u) | (spread4((p1 >> (4 * w)) & 15u) << 1);
    const uint32_t s2 =
        spread4((c2lo >> (4 * w)) & 15u) | (spread4((c2hi >> (4 * w)) & 15u) << 1);
    const uint32_t to_level2 = s1 & (s1 >> 1) & 0x01010101u;  // level-1 code 3
    ew[w] = byte_perm(a.table[2], a.table[0], s1 + to_level2 + s2);
  }
  // Level-3 and raw exponents, in value order.
  {
    uint64_t c = codes3;
    int rank = rr;
    for (uint32_t m = esc2; m; m &= m - 1, c >>= 4) {
      const int k = __builtin_ctz(m);
      const uint32_t code = static_cast<uint32_t>(c) & 15u;
      uint32_t e;
      if (code != 15u) {  // table[16 + code] into byte 0, zeros above
        const uint32_t sel = 0x0c0c0c00u | (code & 7u);
        e = code < 8u ? byte_perm(a.table[5], a.table[4], sel)
                      : byte_perm(a.table[7], a.table[6], sel);
      } else {
        e = rank < lr ? a.raw[rank] : 0u;
        ++rank;
      }
      const int sh = 8 * (k & 3);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t mask = (k >> 2) == w ? 0xffu << sh : 0u;
        ew[w] = (ew[w] & ~mask) | ((e << sh) & mask);
      }
    }
  }
  uint32_t w16[8];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t lo = (sw[w] & 0x7f7f7f7fu) | ((ew[w] << 7) & 0x80808080u);
    const uint32_t hi = (sw[w] & 0x80808080u) | ((ew[w] >> 1) & 0x7f7f7f7fu);
    w16[2 * w] = byte_perm(hi, lo, 0x05010400u);      // values 4w, 4w+1
    w16[2 * w + 1] = byte_perm(hi, lo, 0x07030602u);  // values 4w+2, 4w+3
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

bool counts_valid(int64_t n, int64_t n2, int64_t n3, int64_t nr) {
  return n >= 0 && nr >= 0 && nr <= n3 && n3 <= n2 && n2 <= n;
}

}  // namespace

extern "C" int64_t sf_expert_record_bytes(int64_t n_values, int64_t n_second, int64_t n_third,
                                          int64_t n_raw) {
  if (!counts_valid(n_values, n_second, n_third, n_raw)) return -1;
  return layout(n_values, n_second, n_third, n_raw).total;
}

extern "C" int sf_expert_decode(const void* record, size_t record_bytes, int64_t n_values,
                                const uint8_t* exponent_table, int n_second, int n_third,
                                int n_raw, void* out, sf_stream_t stream) {
  if (!counts_valid(n_values, n_second, n_third, n_raw) || n_values > 0xffffffffLL)
    return SF_ERR_INVALID_ARGUMENT;
  if (n_values == 0) return SF_OK;
  if (!record || !exponent_table || !out) return SF_ERR_INVALID_ARGUMENT;
  const Layout l = layout(n_values, n_second, n_third, n_raw);
  if (static_cast<int64_t>(record_bytes) < l.total) return SF_ERR_INVALID_ARGUMENT;
  if (!aligned16(record) || !aligned16(out)) return SF_ERR_MISALIGNED;
  const uint8_t* base = static_cast<const uint8_t*>(record);
  DecodeArgs a{};
  a.sm = base;
  a.planes = reinterpret_cast<const uint16_t*>(base + l.plane);
  a.plane_words = align256(2 * ((n_values + 15) / 16)) / 2;
  a.l2 = reinterpret_cast<const uint32_t*>(base + l.l2);
  a.l3 = reinterpret_cast<const uint32_t*>(base + l.l3);
  a.raw = base + l.r;
  a.c2 = reinterpret_cast<const uint32_t*>(base + l.c2);
  a.c3 = reinterpret_cast<const uint32_t*>(base + l.c3);
  a.cr = reinterpret_cast<const uint32_t*>(base + l.cr);
  a.out = static_cast<uint16_t*>(out);
  a.n = n_values;
  a.n2 = n_second;
  a.n3 = n_third;
  a.nr = n_raw;
  for (int c = 0; c < 32; ++c)
    a.table[c >> 2] |= static_cast<uint32_t>(exponent_table[c]) << (8 * (c & 3));
  const int64_t blocks = (n_values + kChunk - 1) / kChunk;
  decode_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                  reinterpret_cast<hipStream_t>(stream)>>>(a);
  SF_LAUNCH_CHECK();
  return SF_OK;
}
