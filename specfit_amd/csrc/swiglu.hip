// K3: grouped SwiGLU expert MLP for the verification path on gfx950.
// Restates _expert_forward and the routing-weight scale of the reference
// (src/specfit/runtime/qwen3_offloaded_experts.py:38-62, 132-138, 186-198):
//   gu  = bf16(x . GU^T), act = bf16(bf16(silu(gate)) * up),
//   y   = bf16(act . D^T), row = bf16(y * w_route)
// with GU = packed[0:2IH] as [2I, H] and D = packed[2IH:] as [H, I].
//
// At verification sizes an expert sees m <= a few dozen rows, so each weight
// element is used m times and the GEMMs are bound by streaming the expert's
// weights (9 MiB for Qwen3-30B-A3B) from HBM.  Every weight byte is read from HBM once.
//
// Weight stream.  A workgroup owns a slab of 32 weight rows in a wide launch
// (phase 1: the 16 gate + 16 up rows of 16 activation columns; phase 2: 32
// rows of D, i.e. 32 output columns) or 16 in a narrow one (8 + 8 rows of 8
// columns; 16 rows of D), and streams it in blocks of 256 k.  A block is loaded
// row-contiguously (2 rows x 512 B per wavefront instruction, ~6.2 TB/s on
// MI355X, where loading MFMA B fragments directly touches 16 rows x 64 B per
// instruction and streams at ~4.4 TB/s), two blocks ahead into registers,
// then written to one of two row-padded LDS tiles (16 B of padding per row
// keeps the fragment reads conflict-free) and read back as MFMA B fragments.
// Token rows (the A operand, a few KiB, L2 resident) are loaded straight into
// registers two blocks ahead, each block's right after the MFMAs that used
// the previous contents: in MFMA fragment layout, except in gate/up's split
// for 33..64 rows, which loads them row-contiguously and passes them through
// a per-wavefront LDS region (see mfma_block_staged).  The block count is a
// compile-time constant of the expert shape (built for the Qwen3-30B-A3B and
// Qwen3-235B-A22B experts), so the loop is unrolled and every load is
// unconditional: the compiler's vector-memory wait counts are then exact
// (they are in-order counters; a conditional load would force a full drain).
// Scheduling barriers keep the loads in issue order, so registers hold only
// the blocks in flight.
//
// Work split of a pass.  The 4 wavefronts cover TM sixteen-row token tiles x
// KS k-slices (TM * KS = 4), chosen per workgroup from its expert's row
// count m: m <= 16 -> 1 x 4, m <= 32 -> 2 x 2, larger -> 4 x 1 (two tiles per
// wavefront, 128 rows per pass, for experts above 64 rows).  K-slice partial
// sums are added in LDS in slice order.  So the fp32 summation order of an
// output depends only on (H, I) and the expert's own m, never on the launch,
// its grouping or its other experts.  The kernels are built per row class
// (the launch's largest expert has <= 16 / 32 / 64 / more rows), so a launch
// of small experts runs with the registers of the small split and more
// workgroups per CU.  Rows past the end of a pass repeat the pass's last
// row: an MFMA output row depends only on its own A row and such rows are
// never stored, so loads need no per-lane branches.
// MFMA: v_mfma_f32_16x16x32_bf16, A = token rows (M), B = weight rows (N).
#include <mutex>

#include "sf_common.h"

namespace {

constexpr int kMaxListExperts = 128;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / SF_WAVE;
constexpr int kBlockK = 256;           // k per staged weight block
constexpr int kRowBytes = kBlockK * 2 + 16;  // padded LDS row (bytes)

enum class Resolve { kList, kTable, kDense };

struct SwigluArgs {
  const uint16_t* hidden;
  const int32_t* perm_pos;  // nullptr in dense mode
  const int32_t* offsets;   // nullptr in dense mode
  const uint16_t* route_w;  // nullptr: no routing-weight scale
  uint16_t* act;
  uint16_t* out;
  int64_t row_stride;  // elements between consecutive hidden rows
  int top_k;
  int H;
  int I;
  int dense_m;
  int n;  // list length (list/dense) or number of experts (table)
  const int32_t* slot_of_expert;
  const uint16_t* slot_base;
  int64_t slot_stride;
  int32_t expert[kMaxListExperts];
  uint64_t wptr[kMaxListExperts];
  // List mode with rows_known: first permuted row and row count of each
  // listed expert, so a workgroup starts its weight stream without first
  // reading offsets from memory.
  int rows_known;
  int32_t row0[kMaxListExperts];
  int32_t rows[kMaxListExperts];
};

struct ExpertWork {
  const uint16_t* w;  // packed weights
  int r0;             // first permuted row
  int m;              // rows
};

template <Resolve R>
__device__ __forceinline__ bool resolve(const SwigluArgs& a, int j, ExpertWork& wk) {
  if (R == Resolve::kDense) {
    wk.w = reinterpret_cast<const uint16_t*>(a.wptr[0]);
    wk.r0 = 0;
    wk.m = a.dense_m;
    return wk.m > 0;
  }
  int e;
  if (R == Resolve::kList) {
    wk.w = reinterpret_cast<const uint16_t*>(a.wptr[j]);
    if (a.rows_known) {
      wk.r0 = a.row0[j];
      wk.m = a.rows[j];
      return wk.m > 0;
    }
    e = a.expert[j];
  } else {
    e = j;
    const int slot = a.slot_of_expert[e];
    if (slot < 0) return false;
    wk.w = a.slot_base + static_cast<int64_t>(slot) * a.slot_stride;
  }
  wk.r0 = a.offsets[e];
  wk.m = a.offsets[e + 1] - wk.r0;
  return wk.m > 0;
}

template <Resolve R>
__device__ __forceinline__ const uint16_t* row_ptr(const SwigluArgs& a, int r) {
  if (R == Resolve::kDense) return a.hidden + static_cast<int64_t>(r) * a.row_stride;
  const int tok = a.perm_pos[r] / a.top_k;
  return a.hidden + static_cast<int64_t>(tok) * a.row_stride;
}

// row_ptr in two steps: token_fetch issues the load of permuted row r's
// route position (dense mode: r itself), token_ptr turns the value into the
// token's hidden row.
template <Resolve R>
__device__ __forceinline__ int token_fetch(const SwigluArgs& a, int r) {
  return R == Resolve::kDense ? r : a.perm_pos[r];
}

template <Resolve R>
__device__ __forceinline__ const uint16_t* token_ptr(const SwigluArgs& a, int v) {
  const int tok = R == Resolve::kDense ? v : v / a.top_k;
  return a.hidden + static_cast<int64_t>(tok) * a.row_stride;
}

__device__ __forceinline__ sf_bf16x8 as_bf16x8(uint4 v) {
  return __builtin_bit_cast(sf_bf16x8, v);
}

// Global-memory 16-byte load.  The explicit global address space keeps the
// load a global_load (a flat load also counts against the LDS counter, which
// forces full drains at every LDS wait).
typedef unsigned int sf_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16(const uint16_t* p) {
  const sf_u32x4 v = *(const __attribute__((address_space(1))) sf_u32x4*)(p);
  return __builtin_bit_cast(uint4, v);
}

__device__ __forceinline__ sf_f32x4 mfma16(uint4 a, uint4 b, sf_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}


// ------------------------------------------------------ streaming core --
constexpr int kSteps = kBlockK / 32;  // MFMA k-steps per block
// Blocks in flight ahead of the one in use: 2, and 3 for down's <= 16-row
// split (KS = 4), whose slab is only I / 256 blocks long (3 at I = 768), so
// its workgroups issue every load at the start (16-token all-resident
// launch: down 45.6 -> 44.9 us over the slot table, 49.9 -> 47.6 us over
// listed experts).  Measured slower elsewhere: gate/up at 3 (83.7 -> 85.5
// us), and down's wider splits at 3 (64-token all-resident down 33.9 -> 39.3
// us: their A fragments of a third block cost registers).
// Down's two-tile split (experts above 64 rows) loads its activation rows
// one block ahead instead: with two A tiles per wavefront a second block of
// them held 238 registers, one workgroup per CU; at one block ahead it holds
// 174, two per CU (launches of 12-48 such experts: down 15-29% faster).
constexpr int kDepth = 2;
constexpr int kDownDepth = 3;
constexpr int kGateUpDepth = 2;  // 4 measured no faster (class 1 at 84 experts 6% slower)

// Keeps the compiler's scheduler from moving instructions across this point,
// so loads stay in issue order and registers hold only blocks in flight.
#define SF_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

// A weight slab of 16*NT rows in 8-row blocks: rows 8i .. 8i+7 start at
// part[i] and are `stride` elements apart.
template <int NT>
struct Slab {
  const uint16_t* part[2 * NT];
  int64_t stride;
};

// Lane l of wavefront w loads 16 B of slab row 8i + 2w + l/32 (i < 2*NT) at
// k 8*(l%32) of block b.
template <int NT>
__device__ __forceinline__ void load_w(const Slab<NT>& w, int b, int lane, int wave,
                                       uint4 (&r)[2 * NT]) {
  const int col = b * kBlockK + (lane & 31) * 8;
  const int64_t row = 2 * wave + (lane >> 5);
#pragma unroll
  for (int i = 0; i < 2 * NT; ++i) r[i] = ld16(w.part[i] + row * w.stride + col);
}

template <int NT>
__device__ __forceinline__ void store_w(char* tile, int lane, int wave, const uint4 (&r)[2 * NT]) {
  const int colb = (lane & 31) * 16;
#pragma unroll
  for (int i = 0; i < 2 * NT; ++i) {
    const int row = 8 * i + 2 * wave + (lane >> 5);
    *reinterpret_cast<uint4*>(tile + row * kRowBytes + colb) = r[i];
  }
}

// MFMA B fragment of k-step s for tile rows [r0, r0 + 16): lane l takes row
// r0 + l%16, k 8*(l/16) .. +7 of the step.
__device__ __forceinline__ uint4 frag_b(const char* tile, int r0, int s, int lane) {
  return *reinterpret_cast<const uint4*>(tile + (r0 + (lane & 15)) * kRowBytes + s * 64 +
                                         (lane >> 4) * 16);
}

// A fragments of the SP k-steps of one block that a wavefront's slice uses.
template <int MTW, int SP>
__device__ __forceinline__ void load_x(const uint16_t* const (&xr)[MTW], int b, int s0,
                                       uint4 (&x)[MTW][SP]) {
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
    for (int s = 0; s < SP; ++s) x[mt][s] = ld16(xr[mt] + b * kBlockK + (s0 + s) * 32);
}

// MFMAs of one block: B fragments are read in groups ahead of their MFMAs
// (the scheduling barrier keeps the group's LDS reads together, so their
// latency is paid once per group).
template <int NT, int MTW, int SP>
__device__ __forceinline__ void mfma_block(const char* tile, int s0, const uint4 (&x)[MTW][SP],
                                           int lane, sf_f32x4 (&acc)[MTW][NT]) {
  constexpr int kGroup = 2 < SP ? 2 : SP;
#pragma unroll
  for (int g = 0; g < SP; g += kGroup) {
    uint4 f[kGroup][NT];
#pragma unroll
    for (int s = 0; s < kGroup; ++s)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) f[s][nt] = frag_b(tile, 16 * nt, s0 + g + s, lane);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < kGroup; ++s)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt) acc[mt][nt] = mfma16(x[mt][g + s], f[s][nt], acc[mt][nt]);
  }
}

// Staged A operand of gate/up's one-tile, full-k split (KS = 1, one 16-row
// tile per wavefront, experts of 33..64 rows).  Loading MFMA A fragments
// straight from memory touches 16 token rows x 64 B per instruction; here a
// wavefront loads its 16 rows row-contiguously instead (4 rows x 256 B per
// instruction: half as many cache lines per byte), writes each half block to
// its own LDS region and reads the fragments back.  The MFMA operands are the
// same values, so the results are the same bits.
constexpr int kStageRowBytes = (kBlockK / 2) * 2 + 16;  // half a block of one row (bytes), padded
constexpr int kStageBytes = 16 * kStageRowBytes;      // one wavefront's region

// Lane l loads 16 B at element 8*(l%16) of the half block j/4 of row
// l/16 + 4*(j%4) of the tile (xr[i] = row l/16 + 4i, offset 8*(l%16)).
__device__ __forceinline__ void load_x_rows(const uint16_t* const (&xr)[4], int b,
                                            uint4 (&x)[1][kSteps]) {
#pragma unroll
  for (int j = 0; j < kSteps; ++j) x[0][j] = ld16(xr[j & 3] + b * kBlockK + (j >> 2) * (kBlockK / 2));
}

template <int NT>
__device__ __forceinline__ void mfma_block_staged(const char* tile, char* stage,
                                                  const uint4 (&x)[1][kSteps], int lane,
                                                  sf_f32x4 (&acc)[1][NT]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<uint4*>(stage + (4 * i + (lane >> 4)) * kStageRowBytes + (lane & 15) * 16) =
          x[0][4 * h + i];
    SF_SCHED_FENCE();
#pragma unroll
    for (int g = 0; g < 4; g += 2) {
      uint4 a[2], f[2][NT];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        a[s] = *reinterpret_cast<const uint4*>(stage + (lane & 15) * kStageRowBytes +
                                               (g + s) * 64 + (lane >> 4) * 16);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) f[s][nt] = frag_b(tile, 16 * nt, 4 * h + g + s, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[0][nt] = mfma16(a[s], f[s][nt], acc[0][nt]);
    }
  }
}

// acc = X . W^T over k-slice `slice` of KS (SP = kSteps/KS k-steps of each of
// the NB blocks).  active: wave-uniform, false when the wavefront's tiles
// have no rows (its A loads then hit one cache line, see a_fetch).
struct NoHook {
  __device__ void operator()() const {}
};

// make_xr(xr) fills the NP token-row pointers of the lane.  With kLateX it
// runs after the weight prologue's loads are issued: the pointers of
// gate/up's token rows depend on route positions loaded from memory, and
// computing them first made every workgroup wait for those loads before it
// requested any weight (the first block then waited for two memory
// latencies in a row).  Without it (down: its rows need no load) the
// prologue interleaves weight and row blocks.
// after_issue runs once the prologue's loads are in flight (the place for
// loads whose results are only needed after the stream, e.g. the epilogue's).
// Weight blocks are loaded DW blocks ahead and token-row blocks DX <= DW
// ahead (the token rows are L2 hits; the weights come from HBM).
template <int NT, int MTW, int KS, int NB, int NP, int DW = kDepth, int DX = kDepth,
          bool kLateX = true, typename MakeXr, typename Hook = NoHook>
__device__ __forceinline__ void stream_gemm(const Slab<NT>& w, const MakeXr& make_xr,
                                            int slice, bool active, char* smem, char* stage,
                                            sf_f32x4 (&acc)[MTW][NT],
                                            const Hook& after_issue = Hook{}) {
  constexpr bool kStaged = KS == 1 && MTW == 1 && NP == 4;
  static_assert(NB >= DW && DW >= DX, "prefetch depths exceed the block count");
  constexpr int SP = kSteps / KS;
  constexpr int kTile = 16 * NT * kRowBytes;
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int s0 = slice * SP;
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = sf_f32x4{0.f, 0.f, 0.f, 0.f};
  uint4 wr[DW][2 * NT];
  uint4 xq[DX][MTW][SP];
  const uint16_t* xr[NP];
  if constexpr (kLateX) {
#pragma unroll
    for (int d = 0; d < DW; ++d) load_w<NT>(w, d, lane, wave, wr[d]);
    SF_SCHED_FENCE();
    make_xr(xr);
#pragma unroll
    for (int d = 0; d < DX; ++d) {
      if constexpr (kStaged) load_x_rows(xr, d, xq[d]);
      else load_x<MTW, SP>(xr, d, s0, xq[d]);
    }
  } else {
    make_xr(xr);
#pragma unroll
    for (int d = 0; d < DW; ++d) {
      load_w<NT>(w, d, lane, wave, wr[d]);
      if (d < DX) {
        if constexpr (kStaged) load_x_rows(xr, d, xq[d]);
        else load_x<MTW, SP>(xr, d, s0, xq[d]);
      }
    }
  }
  SF_SCHED_FENCE();
  after_issue();
  SF_SCHED_FENCE();
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int dw = b % DW;
    const int dx = b % DX;
    char* tile = smem + (b & 1) * kTile;
    store_w<NT>(tile, lane, wave, wr[dw]);
    SF_SCHED_FENCE();
    if (b + DW < NB) load_w<NT>(w, b + DW, lane, wave, wr[dw]);
    SF_SCHED_FENCE();
    __syncthreads();  // tile b visible; tile b-1's reads are done
    if constexpr (kStaged) {
      if (active) mfma_block_staged<NT>(tile, stage, xq[dx], lane, acc);
    } else {
      if (active) mfma_block<NT, MTW, SP>(tile, s0, xq[dx], lane, acc);
    }
    SF_SCHED_FENCE();
    if (b + DX < NB) {
      if constexpr (kStaged) load_x_rows(xr, b + DX, xq[dx]);
      else load_x<MTW, SP>(xr, b + DX, s0, xq[dx]);
    }
    SF_SCHED_FENCE();
  }
  __syncthreads();  // the tiles are free again
}

// Adds the KS k-slice partial sums of each tile in slice order, in LDS.
// Returns true for the wavefront that holds the total (slice 0).
template <int NT, int KS>
__device__ __forceinline__ bool reduce_slices(sf_f32x4 (&acc)[1][NT], char* smem) {
  if (KS == 1) return true;
  constexpr int TM = kWaves / KS;
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int t = wave % TM;
  const int q = wave / TM;
  float* part = reinterpret_cast<float*>(smem);  // [KS][TM][NT][4][64], lane-major
  if (q > 0) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[(((q * TM + t) * NT + nt) * 4 + i) * 64 + lane] = acc[0][nt][i];
  }
  __syncthreads();
  if (q == 0) {
#pragma unroll
    for (int qq = 1; qq < KS; ++qq)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[0][nt][i] += part[(((qq * TM + t) * NT + nt) * 4 + i) * 64 + lane];
  }
  __syncthreads();
  return q == 0;
}

// A rows of a wavefront, in two steps.  a_fetch issues fetch(row) for the
// lane's rows (tile mt*TM + wave%TM of the pass, row 16*tile + l%16 clamped
// to the pass; an idle wavefront takes the pass's first row): for gate/up
// that loads the route position of the permuted row.  The values are turned
// into pointers only inside stream_gemm, after its weight prologue is issued
// (fragment_ptrs: + the lane's k offset; an idle wavefront points every
// lane at one address).
template <int MTW, int TM, typename Fetch>
__device__ __forceinline__ bool a_fetch(Fetch fetch, int mp, int (&pre)[MTW]) {
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int t0 = wave % TM;
  const bool active = t0 * 16 < mp;
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt)
    pre[mt] = fetch(active ? min((mt * TM + t0) * 16 + (lane & 15), mp - 1) : 0);
  return active;
}

template <int MTW, typename Ptr>
__device__ __forceinline__ void fragment_ptrs(Ptr ptr, const int (&pre)[MTW], bool active,
                                              const uint16_t* (&xr)[MTW]) {
  const int lane = threadIdx.x & (SF_WAVE - 1);
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt) xr[mt] = ptr(pre[mt]) + (active ? 8 * (lane >> 4) : 0);
}

// Rows of the staged split: lane l holds rows l/16 + 4i (i < 4) of the
// wavefront's tile, clamped to the pass (an idle wavefront: the pass's first
// row); its pointers (staged_ptrs) are at element 8*(l%16).
template <typename Fetch>
__device__ __forceinline__ bool a_fetch_staged(Fetch fetch, int mp, int (&pre)[4]) {
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const bool active = wave * 16 < mp;
#pragma unroll
  for (int i = 0; i < 4; ++i) pre[i] = fetch(active ? min(wave * 16 + (lane >> 4) + 4 * i, mp - 1) : 0);
  return active;
}

template <typename Ptr>
__device__ __forceinline__ void staged_ptrs(Ptr ptr, const int (&pre)[4],
                                            const uint16_t* (&xr)[4]) {
  const int lane = threadIdx.x & (SF_WAVE - 1);
#pragma unroll
  for (int i = 0; i < 4; ++i) xr[i] = ptr(pre[i]) + 8 * (lane & 15);
}

// ---------------------------------------------------------------- phase 1 --
// Workgroup: 8*NT activation columns c0.. of one expert = gate rows c0.. and
// up rows I + c0.. of GU.  NT = 2: the gate and the up rows fill one 16-wide
// MFMA tile each.  NT = 1: one tile holds 8 gate rows then 8 up rows, and
// lane j < 8 of a row takes the up value from lane j + 8 (a DPP row shift).
template <Resolve R, int MTW, int KS, int NB, int NT>
__device__ __forceinline__ void gateup_body(const SwigluArgs& a, const ExpertWork& wk, int tile,
                                            char* smem) {
  constexpr int TM = kWaves / KS;
  constexpr int kPass = 16 * TM * MTW;
  constexpr int kCols = 8 * NT;
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int H = a.H;
  const int c0 = tile * kCols;
  const uint16_t* g = wk.w + static_cast<int64_t>(c0) * H;
  const uint16_t* u = wk.w + static_cast<int64_t>(a.I + c0) * H;
  Slab<NT> w;
  if constexpr (NT == 2) {
    w.part[0] = g;
    w.part[1] = g + static_cast<int64_t>(8) * H;
    w.part[2] = u;
    w.part[3] = u + static_cast<int64_t>(8) * H;
  } else {
    w.part[0] = g;
    w.part[1] = u;
  }
  w.stride = H;
  for (int p0 = 0; p0 < wk.m; p0 += kPass) {
    const int mp = min(kPass, wk.m - p0);
    sf_f32x4 acc[MTW][NT];
    const int base = wk.r0 + p0;
    auto fetch = [&](int row) { return token_fetch<R>(a, base + row); };
    auto ptr = [&](int v) { return token_ptr<R>(a, v); };
    if constexpr (KS == 1 && MTW == 1) {
      int pre[4];
      const bool active = a_fetch_staged(fetch, mp, pre);
      SF_SCHED_FENCE();
      stream_gemm<NT, MTW, KS, NB, 4, kGateUpDepth, kGateUpDepth>(
          w, [&](const uint16_t* (&xr)[4]) { staged_ptrs(ptr, pre, xr); }, 0, active, smem,
          smem + 2 * 16 * NT * kRowBytes + wave * kStageBytes, acc);
    } else {
      int pre[MTW];
      const bool active = a_fetch<MTW, TM>(fetch, mp, pre);
      SF_SCHED_FENCE();
      stream_gemm<NT, MTW, KS, NB, MTW, kGateUpDepth, kGateUpDepth>(
          w, [&](const uint16_t* (&xr)[MTW]) { fragment_ptrs<MTW>(ptr, pre, active, xr); },
          wave / TM, active, smem, nullptr, acc);
    }
    bool owner = true;
    if constexpr (KS > 1) owner = reduce_slices<NT, KS>(acc, smem);
    if (!owner) continue;
    // D layout: lane holds rows 4*(lane/16)+i, column lane%16.
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = (mt * TM + wave % TM) * 16 + 4 * (lane >> 4) + i;
        float gv, uv;
        if constexpr (NT == 2) {
          gv = acc[mt][0][i];
          uv = acc[mt][1][i];
        } else {
          gv = acc[mt][0][i];
          uv = sf_dpp<0x108>(gv);  // row_shl 8: lane j <- lane j + 8
        }
        if (row < mp && (NT == 2 || (lane & 15) < 8)) {
          const float gb = sf_round_bf16(gv);
          const float ub = sf_round_bf16(uv);
          const float sb = sf_round_bf16(sf_silu(gb));
          a.act[static_cast<int64_t>(wk.r0 + p0 + row) * a.I + c0 + (lane & 15)] =
              sf_f32_to_bf16(sb * ub);
        }
      }
    }
  }
}

// Waves per SIMD a build must keep at the Qwen3-30B-A3B shape (gate/up 8
// blocks per row, down 3; list and slot-table launches): the occupancy its
// tiling was measured at.  Several builds sit a register or two under the
// limit of their occupancy, so without the floor a small code change could
// cost each CU a workgroup (gate/up and down of 33..64-row launches hold 3
// workgroups per CU at <= 168 registers).  Other shapes and the one-expert
// form take the compiler's choice.
template <Resolve R, int MC, int NB, int NT>
constexpr int min_waves() {
  if (R == Resolve::kDense || (NB != 8 && NB != 3) || MC == 3) return 1;
  if (NT == 2) return MC == 0 ? 4 : 3;
  return MC == 0 ? (NB == 8 ? 7 : 5) : 1;
}

// Row class MC of a build: 0: every expert of the launch has m <= 16, 1:
// <= 32, 2: <= 64, 3: any.  An expert above its launch's class (max_rows
// understated) runs in passes of the class's largest split.
template <Resolve R, int MC, int NB, int NT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(
    min_waves<R, MC, NB, NT>()))) void gateup_mfma_kernel(const SwigluArgs a) {
  __shared__ __attribute__((aligned(16)))
  char smem[2 * 16 * NT * kRowBytes + (MC >= 2 ? kWaves * kStageBytes : 0)];
  const int tiles = a.I / (8 * NT);
  const int j = blockIdx.x / tiles;
  const int tile = blockIdx.x - j * tiles;
  ExpertWork wk;
  if (!resolve<R>(a, j, wk)) return;
  if (MC == 0 || wk.m <= 16)
    gateup_body<R, 1, 4, NB, NT>(a, wk, tile, smem);
  else if (MC == 1 || wk.m <= 32)
    gateup_body<R, 1, 2, NB, NT>(a, wk, tile, smem);
  else if (MC == 3 && wk.m > 64)
    gateup_body<R, 2, 1, NB, NT>(a, wk, tile, smem);
  else
    gateup_body<R, 1, 1, NB, NT>(a, wk, tile, smem);
}

// ---------------------------------------------------------------- phase 2 --
// Workgroup: 16*NT output columns n0.. of one expert over the full I.
template <Resolve R, int MTW, int KS, int NB, int NT>
__device__ __forceinline__ void down_body(const SwigluArgs& a, const ExpertWork& wk, int tile,
                                          char* smem) {
  constexpr int TM = kWaves / KS;
  constexpr int kPass = 16 * TM * MTW;
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int I = a.I;
  const int n0 = tile * 16 * NT;
  Slab<NT> w;
  const uint16_t* wd = wk.w + 2 * static_cast<int64_t>(a.I) * a.H + static_cast<int64_t>(n0) * I;
#pragma unroll
  for (int h = 0; h < 2 * NT; ++h) w.part[h] = wd + static_cast<int64_t>(8 * h) * I;
  w.stride = I;
  for (int p0 = 0; p0 < wk.m; p0 += kPass) {
    const int mp = min(kPass, wk.m - p0);
    int pre[MTW];
    const bool active = a_fetch<MTW, TM>([&](int row) { return wk.r0 + p0 + row; }, mp, pre);
    const uint16_t* ar[MTW];
    fragment_ptrs<MTW>([&](int r) { return a.act + static_cast<int64_t>(r) * I; }, pre, active,
                       ar);
    auto act_rows = [&](const uint16_t* (&xr)[MTW]) {
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) xr[mt] = ar[mt];
    };
    // Routing weights of this lane's output rows.  The epilogue used to
    // read perm_pos and then route_w for each row after the stream (two
    // dependent global latencies per row at the end of a short workgroup);
    // here perm_pos is read before the stream's first loads and route_w
    // right after them, so both latencies overlap the weight stream.
    int pos[MTW][4];
    float rw[MTW][4];
    const bool scaled = a.route_w != nullptr;
    if (scaled) {
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = min((mt * TM + wave % TM) * 16 + 4 * (lane >> 4) + i, mp - 1);
          pos[mt][i] = a.perm_pos[wk.r0 + p0 + row];
        }
    }
    SF_SCHED_FENCE();
    sf_f32x4 acc[MTW][NT];
    stream_gemm<NT, MTW, KS, NB, MTW, (NB < kDownDepth ? NB : kDownDepth),
                (KS == 4 && NB >= kDownDepth ? kDownDepth : (MTW == 2 ? 1 : kDepth)), false>(
        w, act_rows, wave / TM, active, smem, nullptr, acc, [&] {
          if (scaled) {
#pragma unroll
            for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
              for (int i = 0; i < 4; ++i) rw[mt][i] = sf_bf16_to_f32(a.route_w[pos[mt][i]]);
          }
        });
    bool owner = true;
    if constexpr (KS > 1) owner = reduce_slices<NT, KS>(acc, smem);
    if (!owner) continue;
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = (mt * TM + wave % TM) * 16 + 4 * (lane >> 4) + i;
        if (row < mp) {
          const int r = wk.r0 + p0 + row;
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            float y = sf_round_bf16(acc[mt][nt][i]);
            if (scaled) y = y * rw[mt][i];
            a.out[static_cast<int64_t>(r) * a.H + n0 + 16 * nt + (lane & 15)] = sf_f32_to_bf16(y);
          }
        }
      }
    }
  }
}

template <Resolve R, int MC, int NB, int NT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(
    min_waves<R, MC, NB, NT>()))) void down_mfma_kernel(const SwigluArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[2 * 16 * NT * kRowBytes];
  const int tiles = a.H / (16 * NT);
  const int j = blockIdx.x / tiles;
  const int tile = blockIdx.x - j * tiles;
  ExpertWork wk;
  if (!resolve<R>(a, j, wk)) return;
  if (MC == 0 || wk.m <= 16)
    down_body<R, 1, 4, NB, NT>(a, wk, tile, smem);
  else if (MC == 1 || wk.m <= 32)
    down_body<R, 1, 2, NB, NT>(a, wk, tile, smem);
  else if (MC == 3 && wk.m > 64)
    down_body<R, 2, 1, NB, NT>(a, wk, tile, smem);
  else
    down_body<R, 1, 1, NB, NT>(a, wk, tile, smem);
}

// ------------------------------------------------ generic (any shape) path --
// One workgroup per expert; plain fp32 loops in ascending k.  Used for shapes
// the MFMA tiling does not cover (tiny test models); same rounding points.
template <Resolve R>
__global__ __launch_bounds__(kThreads) void gateup_generic_kernel(const SwigluArgs a) {
  ExpertWork wk;
  if (!resolve<R>(a, blockIdx.x, wk)) return;
  const int H = a.H, I = a.I;
  for (int q = threadIdx.x; q < wk.m * I; q += kThreads) {
    const int row = q / I;
    const int c = q - row * I;
    const uint16_t* x = row_ptr<R>(a, wk.r0 + row);
    const uint16_t* g = wk.w + static_cast<int64_t>(c) * H;
    const uint16_t* u = wk.w + static_cast<int64_t>(I + c) * H;
    float ga = 0.f, ua = 0.f;
    for (int k = 0; k < H; ++k) {
      const float xv = sf_bf16_to_f32(x[k]);
      ga = __builtin_fmaf(xv, sf_bf16_to_f32(g[k]), ga);
      ua = __builtin_fmaf(xv, sf_bf16_to_f32(u[k]), ua);
    }
    const float gb = sf_round_bf16(ga);
    const float ub = sf_round_bf16(ua);
    const float sb = sf_round_bf16(sf_silu(gb));
    a.act[static_cast<int64_t>(wk.r0 + row) * I + c] = sf_f32_to_bf16(sb * ub);
  }
}

template <Resolve R>
__global__ __launch_bounds__(kThreads) void down_generic_kernel(const SwigluArgs a) {
  ExpertWork wk;
  if (!resolve<R>(a, blockIdx.x, wk)) return;
  const int H = a.H, I = a.I;
  const uint16_t* d = wk.w + 2 * static_cast<int64_t>(I) * H;
  for (int q = threadIdx.x; q < wk.m * H; q += kThreads) {
    const int row = q / H;
    const int n = q - row * H;
    const int r = wk.r0 + row;
    const uint16_t* x = a.act + static_cast<int64_t>(r) * I;
    const uint16_t* dn = d + static_cast<int64_t>(n) * I;
    float acc = 0.f;
    for (int k = 0; k < I; ++k)
      acc = __builtin_fmaf(sf_bf16_to_f32(x[k]), sf_bf16_to_f32(dn[k]), acc);
    float y = sf_round_bf16(acc);
    if (a.route_w) y = y * sf_bf16_to_f32(a.route_w[a.perm_pos[r]]);
    a.out[static_cast<int64_t>(r) * H + n] = sf_f32_to_bf16(y);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compiled (H, I) shapes of the MFMA path, as 256-k block counts of a
// gate/up row (H / 256) and of a down row (I / 256): the Qwen3-30B-A3B
// expert (H = 2048, I = 768) and the Qwen3-235B-A22B expert (H = 4096,
// I = 1536).  Other shapes take the generic kernels.
enum class Shape { kGeneric, k2048x768, k4096x1536 };

Shape mfma_shape(int H, int I) {
  if (H == 8 * kBlockK && I == 3 * kBlockK) return Shape::k2048x768;
  if (H == 16 * kBlockK && I == 6 * kBlockK) return Shape::k4096x1536;
  return Shape::kGeneric;
}

template <Resolve R, int MC, int NT, int NBG, int NBD>
int launch_mfma(const SwigluArgs& a, int groups, hipStream_t s) {
  const long long g1 = static_cast<long long>(groups) * (a.I / (8 * NT));
  const long long g2 = static_cast<long long>(groups) * (a.H / (16 * NT));
  if (g1 > 0x7fffffffLL || g2 > 0x7fffffffLL) return SF_ERR_UNSUPPORTED_SHAPE;
  gateup_mfma_kernel<R, MC, NBG, NT><<<dim3(static_cast<unsigned>(g1)), dim3(kThreads), 0, s>>>(a);
  SF_LAUNCH_CHECK();
  down_mfma_kernel<R, MC, NBD, NT><<<dim3(static_cast<unsigned>(g2)), dim3(kThreads), 0, s>>>(a);
  SF_LAUNCH_CHECK();
  return SF_OK;
}

// Tile width.  A narrow launch (8 activation columns per gate/up workgroup,
// 16 output columns per down workgroup) has twice the workgroups of a wide
// one (16 / 32), so a launch of few small experts covers more CUs; each of
// its workgroups re-reads the expert's token rows, so the narrow form costs
// more than it gains once a launch carries many experts or experts of more
// than 16 rows.  Measured on MI355X at the Qwen3-30B-A3B shape: 1-4 experts
// of <= 16 rows run 10-15% faster narrow, ~120 experts of <= 16 rows 2%
// slower, 12 experts of <= 64 rows no faster when their weights were just
// copied in.  Both widths give bit-identical results: a column's summation
// order does not depend on the tile it sits in.
constexpr int kNarrowMaxGroups = 24;

bool narrow_tiles(int groups, int max_rows) {
  return max_rows <= 16 && groups <= kNarrowMaxGroups;
}

template <Resolve R, int NT, int NBG, int NBD>
int launch_class(const SwigluArgs& a, int groups, int max_rows, hipStream_t s) {
  if (max_rows <= 16) return launch_mfma<R, 0, NT, NBG, NBD>(a, groups, s);
  if (max_rows <= 32) return launch_mfma<R, 1, NT, NBG, NBD>(a, groups, s);
  if (max_rows <= 64) return launch_mfma<R, 2, NT, NBG, NBD>(a, groups, s);
  return launch_mfma<R, 3, NT, NBG, NBD>(a, groups, s);
}

template <Resolve R, int NBG, int NBD>
int launch_width(const SwigluArgs& a, int groups, int max_rows, hipStream_t s) {
  if (narrow_tiles(groups, max_rows)) return launch_class<R, 1, NBG, NBD>(a, groups, max_rows, s);
  return launch_class<R, 2, NBG, NBD>(a, groups, max_rows, s);
}

// max_rows bounds the rows of any expert of the launch; it picks the row
// class of the build.
template <Resolve R>
int launch(const SwigluArgs& a, int groups, Shape shape, int max_rows, hipStream_t s) {
  if (groups <= 0) return SF_OK;
  if (shape == Shape::k2048x768) return launch_width<R, 8, 3>(a, groups, max_rows, s);
  if (shape == Shape::k4096x1536) return launch_width<R, 16, 6>(a, groups, max_rows, s);
  gateup_generic_kernel<R><<<dim3(groups), dim3(kThreads), 0, s>>>(a);
  SF_LAUNCH_CHECK();
  down_generic_kernel<R><<<dim3(groups), dim3(kThreads), 0, s>>>(a);
  SF_LAUNCH_CHECK();
  return SF_OK;
}

int check_common(int tokens, int top_k, int H, int I) {
  if (tokens < 0 || top_k < 1 || H < 1 || I < 1) return SF_ERR_INVALID_ARGUMENT;
  if (static_cast<long long>(tokens) * top_k > 0x7fffffffLL) return SF_ERR_UNSUPPORTED_SHAPE;
  return SF_OK;
}

}  // namespace

extern "C" int sf_grouped_swiglu(const void* hidden, const int32_t* perm_pos,
                                 const int32_t* offsets, const void* route_weights,
                                 int tokens, int top_k, int hidden_size,
                                 int intermediate_size, int n_experts, int max_rows,
                                 const int32_t* expert_ids,
                                 const uint64_t* expert_weights,
                                 const int32_t* expert_row_begin,
                                 const int32_t* expert_row_count,
                                 void* act_workspace, void* out_rows,
                                 sf_stream_t stream) {
  int rc = check_common(tokens, top_k, hidden_size, intermediate_size);
  if (rc) return rc;
  if (n_experts < 0 || max_rows < 1) return SF_ERR_INVALID_ARGUMENT;
  if (n_experts == 0 || tokens == 0) return SF_OK;
  if (!hidden || !perm_pos || !offsets || !expert_ids || !expert_weights ||
      !act_workspace || !out_rows)
    return SF_ERR_INVALID_ARGUMENT;
  if ((expert_row_begin == nullptr) != (expert_row_count == nullptr)) return SF_ERR_INVALID_ARGUMENT;
  const bool rows_known = expert_row_begin != nullptr;
  for (int i = 0; rows_known && i < n_experts; ++i) {
    const long long end = static_cast<long long>(expert_row_begin[i]) + expert_row_count[i];
    if (expert_row_begin[i] < 0 || expert_row_count[i] < 0 ||
        end > static_cast<long long>(tokens) * top_k)
      return SF_ERR_INVALID_ARGUMENT;
  }
  bool aligned = aligned16(hidden) && aligned16(act_workspace);
  for (int i = 0; i < n_experts; ++i) {
    if (expert_ids[i] < 0 || expert_weights[i] == 0) return SF_ERR_INVALID_ARGUMENT;
    if (expert_weights[i] & 15u) aligned = false;
  }
  const Shape shape = aligned ? mfma_shape(hidden_size, intermediate_size) : Shape::kGeneric;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  for (int base = 0; base < n_experts; base += kMaxListExperts) {
    SwigluArgs a{};
    a.hidden = static_cast<const uint16_t*>(hidden);
    a.perm_pos = perm_pos;
    a.offsets = offsets;
    a.route_w = static_cast<const uint16_t*>(route_weights);
    a.act = static_cast<uint16_t*>(act_workspace);
    a.out = static_cast<uint16_t*>(out_rows);
    a.row_stride = hidden_size;
    a.top_k = top_k;
    a.H = hidden_size;
    a.I = intermediate_size;
    a.n = n_experts - base < kMaxListExperts ? n_experts - base : kMaxListExperts;
    a.rows_known = rows_known ? 1 : 0;
    for (int i = 0; i < a.n; ++i) {
      a.expert[i] = expert_ids[base + i];
      a.wptr[i] = expert_weights[base + i];
      if (rows_known) {
        a.row0[i] = expert_row_begin[base + i];
        a.rows[i] = expert_row_count[base + i];
      }
    }
    rc = launch<Resolve::kList>(a, a.n, shape, max_rows, s);
    if (rc) return rc;
  }
  return SF_OK;
}

namespace {

// Slot-table launch shared by sf_grouped_swiglu_table and its
// allocation-free variant; `act` is the activation workspace.
int table_launch(const void* hidden, const int32_t* perm_pos, const int32_t* offsets,
                 const void* route_weights, int tokens, int top_k, int hidden_size,
                 int intermediate_size, int num_experts, int max_rows,
                 const int32_t* slot_of_expert, const void* slot_base,
                 int64_t slot_stride_elems, void* act, void* out_rows, hipStream_t stream) {
  const bool aligned = aligned16(hidden) && aligned16(act) && aligned16(slot_base) &&
                       (slot_stride_elems % 8 == 0);
  const Shape shape = aligned ? mfma_shape(hidden_size, intermediate_size) : Shape::kGeneric;
  SwigluArgs a{};
  a.hidden = static_cast<const uint16_t*>(hidden);
  a.perm_pos = perm_pos;
  a.offsets = offsets;
  a.route_w = static_cast<const uint16_t*>(route_weights);
  a.act = static_cast<uint16_t*>(act);
  a.out = static_cast<uint16_t*>(out_rows);
  a.row_stride = hidden_size;
  a.top_k = top_k;
  a.H = hidden_size;
  a.I = intermediate_size;
  a.n = num_experts;
  a.slot_of_expert = slot_of_expert;
  a.slot_base = static_cast<const uint16_t*>(slot_base);
  a.slot_stride = slot_stride_elems;
  return launch<Resolve::kTable>(a, num_experts, shape, max_rows, stream);
}

int check_table(int tokens, int top_k, int hidden_size, int intermediate_size, int num_experts,
                int max_rows, int64_t slot_stride_elems) {
  const int rc = check_common(tokens, top_k, hidden_size, intermediate_size);
  if (rc) return rc;
  if (num_experts < 1 || slot_stride_elems < 0 || max_rows < 1) return SF_ERR_INVALID_ARGUMENT;
  return SF_OK;
}

// ------------------------------------------------ allocation-free variant --
// The activation workspace of sf_grouped_swiglu_table_noalloc lives in this
// fixed device array (one copy per GPU, held until the process ends).  Host
// code never passes `scratch` itself to a kernel: in host code that name is
// a host-side stand-in, so each device's address is looked up once with
// hipGetSymbolAddress and used instead.
constexpr size_t kScratchBytes = SF_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint16_t scratch[kScratchBytes / sizeof(uint16_t)];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t status = hipSuccess;
};

DeviceScratch g_scratch[kMaxDevices];

// Device address of `scratch` on the device of `stream` (the current device
// for the null stream), resolved on that device's first call with the device
// made current for the lookup.
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  const hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return SF_ERR_HIP_BASE + static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return SF_ERR_INVALID_ARGUMENT;
  DeviceScratch& ds = g_scratch[dev];
  std::call_once(ds.once, [&] {
    int current = -1;
    hipError_t st = hipGetDevice(&current);
    if (st == hipSuccess && current != dev) st = hipSetDevice(dev);
    void* p = nullptr;
    if (st == hipSuccess) st = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (current >= 0 && current != dev) {
      const hipError_t back = hipSetDevice(current);
      if (st == hipSuccess) st = back;
    }
    ds.status = st;
    ds.ptr = st == hipSuccess ? p : nullptr;
  });
  if (ds.status != hipSuccess) return SF_ERR_HIP_BASE + static_cast<int>(ds.status);
  *out = ds.ptr;
  return SF_OK;
}

}  // namespace

extern "C" int sf_grouped_swiglu_table(const void* hidden, const int32_t* perm_pos,
                                       const int32_t* offsets, const void* route_weights,
                                       int tokens, int top_k, int hidden_size,
                                       int intermediate_size, int num_experts, int max_rows,
                                       const int32_t* slot_of_expert,
                                       const void* slot_base, int64_t slot_stride_elems,
                                       void* act_workspace, void* out_rows,
                                       sf_stream_t stream) {
  const int rc = check_table(tokens, top_k, hidden_size, intermediate_size, num_experts,
                             max_rows, slot_stride_elems);
  if (rc) return rc;
  if (tokens == 0) return SF_OK;
  if (!hidden || !perm_pos || !offsets || !slot_of_expert || !slot_base ||
      !act_workspace || !out_rows)
    return SF_ERR_INVALID_ARGUMENT;
  return table_launch(hidden, perm_pos, offsets, route_weights, tokens, top_k, hidden_size,
                      intermediate_size, num_experts, max_rows, slot_of_expert, slot_base,
                      slot_stride_elems, act_workspace, out_rows,
                      reinterpret_cast<hipStream_t>(stream));
}

extern "C" int sf_grouped_swiglu_table_noalloc(const void* hidden, const int32_t* perm_pos,
                                               const int32_t* offsets, const void* route_weights,
                                               int tokens, int top_k, int hidden_size,
                                               int intermediate_size, int num_experts,
                                               int max_rows, const int32_t* slot_of_expert,
                                               const void* slot_base, int64_t slot_stride_elems,
                                               void* out_rows, sf_stream_t stream) {
  const int rc = check_table(tokens, top_k, hidden_size, intermediate_size, num_experts,
                             max_rows, slot_stride_elems);
  if (rc) return rc;
  if (tokens == 0) return SF_OK;
  if (!hidden || !perm_pos || !offsets || !slot_of_expert || !slot_base || !out_rows)
    return SF_ERR_INVALID_ARGUMENT;
  const size_t need = static_cast<size_t>(tokens) * static_cast<size_t>(top_k) *
                      static_cast<size_t>(intermediate_size) * sizeof(uint16_t);
  if (need > kScratchBytes) return SF_ERR_SCRATCH_LIMIT;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  void* act = nullptr;
  const int sr = scratch_address(s, &act);
  if (sr) return sr;
  return table_launch(hidden, perm_pos, offsets, route_weights, tokens, top_k, hidden_size,
                      intermediate_size, num_experts, max_rows, slot_of_expert, slot_base,
                      slot_stride_elems, act, out_rows, s);
}

extern "C" int sf_expert_swiglu(const void* rows, int m, int64_t row_stride,
                                int hidden_size, int intermediate_size,
                                const void* packed_weights, void* act_workspace,
                                void* out, sf_stream_t stream) {
  if (m < 0 || hidden_size < 1 || intermediate_size < 1 || row_stride < hidden_size)
    return SF_ERR_INVALID_ARGUMENT;
  if (m == 0) return SF_OK;
  if (!rows || !packed_weights || !act_workspace || !out) return SF_ERR_INVALID_ARGUMENT;
  const bool aligned = aligned16(rows) && (row_stride % 8 == 0) && aligned16(packed_weights) &&
                       aligned16(act_workspace);
  const Shape shape = aligned ? mfma_shape(hidden_size, intermediate_size) : Shape::kGeneric;
  SwigluArgs a{};
  a.hidden = static_cast<const uint16_t*>(rows);
  a.act = static_cast<uint16_t*>(act_workspace);
  a.out = static_cast<uint16_t*>(out);
  a.row_stride = row_stride;
  a.top_k = 1;
  a.H = hidden_size;
  a.I = intermediate_size;
  a.dense_m = m;
  a.n = 1;
  a.wptr[0] = reinterpret_cast<uint64_t>(packed_weights);
  return launch<Resolve::kDense>(a, 1, shape, m, reinterpret_cast<hipStream_t>(stream));
}
