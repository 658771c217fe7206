// K3: grouped SwiGLU expert MLP for the verification path on gfx950.
// Restates _expert_forward and the routing-weight scale of the reference
// (src/specfit/runtime/qwen3_offloaded_experts.py:38-62, 132-138, 186-198):
//   gu  = bf16(x . GU^T), act = bf16(bf16(silu(gate)) * up),
//   y   = bf16(act . D^T), row = bf16(y * w_route)
// with GU = packed[0:2IH] as [2I, H] and D = packed[2IH:] as [H, I].
//
// At verification sizes an expert sees m <= a few dozen rows, so each weight
// element is used m times and the GEMMs are bound by streaming the 9 MiB of
// expert weights from HBM.  Every weight byte is read exactly once.
//
// Weight access pattern.  A 16x16x32 MFMA B operand, loaded directly, touches
// 16 weight rows x 64 B per load instruction; on MI355X that pattern streams
// HBM at ~4.4 TB/s, while row-contiguous 1 KiB loads stream at ~6.2 TB/s.  So
// weights are read as blocks of 2 rows x 512 B per instruction (256 k per
// row), written to a wavefront-private, row-padded LDS tile (16 B of padding
// per row keeps the transposed reads free of bank conflicts) and read back in
// MFMA-operand order.  Token rows (the A operand, a few KiB, L2 resident) are
// loaded straight into registers.
//
// Phase 1 (gate/up): a workgroup owns 16 activation columns of one expert,
// i.e. 16 gate rows + 16 up rows of GU.  Its 4 wavefronts split H into
// quarters; partial tiles are summed in LDS in wavefront order
// (deterministic), then the SwiGLU epilogue writes bf16 activations.
// Phase 2 (down): a workgroup owns 64 output columns (4 wavefronts x 16) of
// one expert over the full I; the epilogue applies the routing weight.
//
// Rows per pass: each workgroup picks 1, 2 or 4 sixteen-row MFMA tiles from
// its own expert's row count (capped by the launch's max_rows), so small
// experts do not pay for the largest expert of a launch.  Rows past the end
// of a pass repeat the pass's last row: an MFMA output row depends only on
// its own A row and rows past the end are never stored, so the loads need
// no per-lane branches.  The fp32 summation order of every output is fixed
// by (H, I) alone, so results do not depend on grouping, tile count or
// launch.
// MFMA: v_mfma_f32_16x16x32_bf16, A = token rows (M), B = weight rows (N).
#include "sf_common.h"

namespace {

constexpr int kMaxListExperts = 128;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / SF_WAVE;
constexpr int kGateCols = 16;          // activation columns per phase-1 workgroup
constexpr int kDownCols = 16 * kWaves; // output columns per phase-2 workgroup
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
    e = a.expert[j];
    wk.w = reinterpret_cast<const uint16_t*>(a.wptr[j]);
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

__device__ __forceinline__ sf_bf16x8 as_bf16x8(uint4 v) {
  return __builtin_bit_cast(sf_bf16x8, v);
}

__device__ __forceinline__ uint4 ld16(const uint16_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

__device__ __forceinline__ sf_f32x4 mfma16(uint4 a, uint4 b, sf_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Stage ROWS (even) weight rows x kBlockK k into a wavefront's LDS tile:
// lane l loads 16 B of row 2i + l/32 at k offset 8*(l%32); row r of the
// block starts at w_row0 + r * row_stride.
template <int ROWS>
__device__ __forceinline__ void stage_block(const uint16_t* w_row0, int64_t row_stride,
                                            char* tile, int lane) {
  const int half = lane >> 5;
  const int col = (lane & 31) * 8;
  uint4 v[ROWS / 2];
#pragma unroll
  for (int i = 0; i < ROWS / 2; ++i)
    v[i] = ld16(w_row0 + static_cast<int64_t>(2 * i + half) * row_stride + col);
#pragma unroll
  for (int i = 0; i < ROWS / 2; ++i)
    *reinterpret_cast<uint4*>(tile + (2 * i + half) * kRowBytes + col * 2) = v[i];
}

// MFMA B fragment of k-step s (32 k) for tile rows [r0, r0 + 16): lane l
// takes row r0 + l%16, k 8*(l/16) .. +7 of the step.
__device__ __forceinline__ uint4 frag_b(const char* tile, int r0, int s, int lane) {
  return *reinterpret_cast<const uint4*>(tile + (r0 + (lane & 15)) * kRowBytes + s * 64 +
                                         (lane >> 4) * 16);
}

// Sixteen-row tiles needed by an expert of m rows, capped at MTMAX.
template <int MTMAX>
__device__ __forceinline__ int tiles_for(int m) {
  return (min(m, 16 * MTMAX) + 15) / 16;
}

// ---------------------------------------------------------------- phase 1 --
template <Resolve R, int MT>
__device__ __forceinline__ void gateup_body(const SwigluArgs& a, const ExpertWork& wk, int tile,
                                            char* smem) {
  constexpr int kRows = 16 * MT;
  auto s_part = reinterpret_cast<float(*)[2][kRows][kGateCols]>(smem);
  auto s_w = reinterpret_cast<char(*)[32 * kRowBytes]>(smem);
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int H = a.H;
  const int c0 = tile * kGateCols;
  const int kq = H / kWaves;
  const int kbeg = wave * kq;
  const int lrow = lane & 15;
  const int kl = 8 * (lane >> 4);
  char* wt = s_w[wave];
  // LDS tile rows 0..15: gate rows c0.., rows 16..31: up rows I + c0..
  const uint16_t* wgate = wk.w + static_cast<int64_t>(c0) * H + kbeg;
  const uint16_t* wup = wk.w + static_cast<int64_t>(a.I + c0) * H + kbeg;
  const int blocks = kq / kBlockK;

  for (int p0 = 0; p0 < wk.m; p0 += kRows) {
    const int mp = min(kRows, wk.m - p0);
    const uint16_t* xr[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      xr[mt] = row_ptr<R>(a, wk.r0 + p0 + min(mt * 16 + lrow, mp - 1)) + kbeg + kl;
    sf_f32x4 acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc[mt][0] = sf_f32x4{0.f, 0.f, 0.f, 0.f};
      acc[mt][1] = sf_f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int b = 0; b < blocks; ++b) {
      stage_block<16>(wgate + b * kBlockK, H, wt, lane);
      stage_block<16>(wup + b * kBlockK, H, wt + 16 * kRowBytes, lane);
#pragma unroll
      for (int s = 0; s < kBlockK / 32; ++s) {
        uint4 x[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) x[mt] = ld16(xr[mt] + b * kBlockK + s * 32);
        const uint4 g = frag_b(wt, 0, s, lane);
        const uint4 u = frag_b(wt, 16, s, lane);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[mt][0] = mfma16(x[mt], g, acc[mt][0]);
          acc[mt][1] = mfma16(x[mt], u, acc[mt][1]);
        }
      }
    }
    __syncthreads();  // every wavefront is done with its weight tile
    // D layout: lane holds rows 4*(lane/16)+i, column lane%16.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = mt * 16 + 4 * (lane >> 4) + i;
        s_part[wave][0][row][lrow] = acc[mt][0][i];
        s_part[wave][1][row][lrow] = acc[mt][1][i];
      }
    }
    __syncthreads();
    for (int q = threadIdx.x; q < mp * kGateCols; q += kThreads) {
      const int row = q / kGateCols;
      const int col = q - row * kGateCols;
      float g = s_part[0][0][row][col];
      float up = s_part[0][1][row][col];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) {
        g += s_part[w][0][row][col];
        up += s_part[w][1][row][col];
      }
      const float gb = sf_round_bf16(g);
      const float ub = sf_round_bf16(up);
      const float sb = sf_round_bf16(sf_silu(gb));
      a.act[static_cast<int64_t>(wk.r0 + p0 + row) * a.I + c0 + col] = sf_f32_to_bf16(sb * ub);
    }
    __syncthreads();
  }
}

template <Resolve R, int MTMAX>
__global__ __launch_bounds__(kThreads) void gateup_mfma_kernel(const SwigluArgs a) {
  // The weight tiles are dead once the K loop ends, so the cross-wavefront
  // partial sums reuse their LDS.
  constexpr int kTileBytes = kWaves * 32 * kRowBytes;
  constexpr int kPartBytes = kWaves * 2 * 16 * MTMAX * kGateCols * 4;
  __shared__ __attribute__((aligned(16))) char smem[kTileBytes > kPartBytes ? kTileBytes : kPartBytes];
  const int tiles = a.I / kGateCols;
  const int j = blockIdx.x / tiles;
  const int tile = blockIdx.x - j * tiles;
  ExpertWork wk;
  if (!resolve<R>(a, j, wk)) return;
  const int need = tiles_for<MTMAX>(wk.m);
  if (MTMAX >= 4 && need > 2)
    gateup_body<R, 4>(a, wk, tile, smem);
  else if (MTMAX >= 2 && need > 1)
    gateup_body<R, 2>(a, wk, tile, smem);
  else
    gateup_body<R, 1>(a, wk, tile, smem);
}

// ---------------------------------------------------------------- phase 2 --
template <Resolve R, int MT>
__device__ __forceinline__ void down_body(const SwigluArgs& a, const ExpertWork& wk, int tile,
                                          char* smem) {
  constexpr int kRows = 16 * MT;
  auto s_w = reinterpret_cast<char(*)[16 * kRowBytes]>(smem);
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int I = a.I;
  const int n0 = tile * kDownCols + wave * 16;
  const int lrow = lane & 15;
  const int kl = 8 * (lane >> 4);
  char* wt = s_w[wave];
  const uint16_t* wd = wk.w + 2 * static_cast<int64_t>(a.I) * a.H + static_cast<int64_t>(n0) * I;
  const int blocks = I / kBlockK;

  for (int p0 = 0; p0 < wk.m; p0 += kRows) {
    const int mp = min(kRows, wk.m - p0);
    const uint16_t* ar[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      ar[mt] = a.act + static_cast<int64_t>(wk.r0 + p0 + min(mt * 16 + lrow, mp - 1)) * I + kl;
    sf_f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = sf_f32x4{0.f, 0.f, 0.f, 0.f};
    for (int b = 0; b < blocks; ++b) {
      stage_block<16>(wd + b * kBlockK, I, wt, lane);
#pragma unroll
      for (int s = 0; s < kBlockK / 32; ++s) {
        uint4 x[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) x[mt] = ld16(ar[mt] + b * kBlockK + s * 32);
        const uint4 d = frag_b(wt, 0, s, lane);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma16(x[mt], d, acc[mt]);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = mt * 16 + 4 * (lane >> 4) + i;
        if (row < mp) {
          const int r = wk.r0 + p0 + row;
          float y = sf_round_bf16(acc[mt][i]);
          if (a.route_w) y = y * sf_bf16_to_f32(a.route_w[a.perm_pos[r]]);
          a.out[static_cast<int64_t>(r) * a.H + n0 + lrow] = sf_f32_to_bf16(y);
        }
      }
    }
  }
}

template <Resolve R, int MTMAX>
__global__ __launch_bounds__(kThreads) void down_mfma_kernel(const SwigluArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kWaves * 16 * kRowBytes];
  const int tiles = a.H / kDownCols;
  const int j = blockIdx.x / tiles;
  const int tile = blockIdx.x - j * tiles;
  ExpertWork wk;
  if (!resolve<R>(a, j, wk)) return;
  const int need = tiles_for<MTMAX>(wk.m);
  if (MTMAX >= 4 && need > 2)
    down_body<R, 4>(a, wk, tile, smem);
  else if (MTMAX >= 2 && need > 1)
    down_body<R, 2>(a, wk, tile, smem);
  else
    down_body<R, 1>(a, wk, tile, smem);
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

bool mfma_shape_ok(int H, int I) {
  // phase 1: each wavefront's K range (H/4) is whole staged blocks; phase 2:
  // I is whole staged blocks and H whole 64-column workgroups.
  return H % (kWaves * kBlockK) == 0 && H % kDownCols == 0 && I % kGateCols == 0 &&
         I % kBlockK == 0;
}

template <Resolve R, int MTMAX>
int launch_mfma(const SwigluArgs& a, long long g1, long long g2, hipStream_t s) {
  gateup_mfma_kernel<R, MTMAX><<<dim3(static_cast<unsigned>(g1)), dim3(kThreads), 0, s>>>(a);
  SF_LAUNCH_CHECK();
  down_mfma_kernel<R, MTMAX><<<dim3(static_cast<unsigned>(g2)), dim3(kThreads), 0, s>>>(a);
  SF_LAUNCH_CHECK();
  return SF_OK;
}

// max_rows bounds the rows of any expert of the launch; it only caps the
// tile count (results do not depend on it).
template <Resolve R>
int launch(const SwigluArgs& a, int groups, bool mfma, int max_rows, hipStream_t s) {
  if (groups <= 0) return SF_OK;
  if (mfma) {
    const long long g1 = static_cast<long long>(groups) * (a.I / kGateCols);
    const long long g2 = static_cast<long long>(groups) * (a.H / kDownCols);
    if (g1 > 0x7fffffffLL || g2 > 0x7fffffffLL) return SF_ERR_UNSUPPORTED_SHAPE;
    if (max_rows <= 16) return launch_mfma<R, 1>(a, g1, g2, s);
    if (max_rows <= 32) return launch_mfma<R, 2>(a, g1, g2, s);
    return launch_mfma<R, 4>(a, g1, g2, s);
  }
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
                                 void* act_workspace, void* out_rows,
                                 sf_stream_t stream) {
  int rc = check_common(tokens, top_k, hidden_size, intermediate_size);
  if (rc) return rc;
  if (n_experts < 0 || max_rows < 1) return SF_ERR_INVALID_ARGUMENT;
  if (n_experts == 0 || tokens == 0) return SF_OK;
  if (!hidden || !perm_pos || !offsets || !expert_ids || !expert_weights ||
      !act_workspace || !out_rows)
    return SF_ERR_INVALID_ARGUMENT;
  bool mfma = mfma_shape_ok(hidden_size, intermediate_size) && aligned16(hidden) &&
              aligned16(act_workspace);
  for (int i = 0; i < n_experts; ++i) {
    if (expert_ids[i] < 0 || expert_weights[i] == 0) return SF_ERR_INVALID_ARGUMENT;
    if (expert_weights[i] & 15u) mfma = false;
  }
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
    for (int i = 0; i < a.n; ++i) {
      a.expert[i] = expert_ids[base + i];
      a.wptr[i] = expert_weights[base + i];
    }
    rc = launch<Resolve::kList>(a, a.n, mfma, max_rows, s);
    if (rc) return rc;
  }
  return SF_OK;
}

extern "C" int sf_grouped_swiglu_table(const void* hidden, const int32_t* perm_pos,
                                       const int32_t* offsets, const void* route_weights,
                                       int tokens, int top_k, int hidden_size,
                                       int intermediate_size, int num_experts,
                                       const int32_t* slot_of_expert,
                                       const void* slot_base, int64_t slot_stride_elems,
                                       void* act_workspace, void* out_rows,
                                       sf_stream_t stream) {
  int rc = check_common(tokens, top_k, hidden_size, intermediate_size);
  if (rc) return rc;
  if (num_experts < 1 || slot_stride_elems < 0) return SF_ERR_INVALID_ARGUMENT;
  if (tokens == 0) return SF_OK;
  if (!hidden || !perm_pos || !offsets || !slot_of_expert || !slot_base ||
      !act_workspace || !out_rows)
    return SF_ERR_INVALID_ARGUMENT;
  const bool mfma = mfma_shape_ok(hidden_size, intermediate_size) && aligned16(hidden) &&
                    aligned16(act_workspace) && aligned16(slot_base) &&
                    (slot_stride_elems % 8 == 0);
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
  a.n = num_experts;
  a.slot_of_expert = slot_of_expert;
  a.slot_base = static_cast<const uint16_t*>(slot_base);
  a.slot_stride = slot_stride_elems;
  return launch<Resolve::kTable>(a, num_experts, mfma, tokens * top_k,
                                 reinterpret_cast<hipStream_t>(stream));
}

extern "C" int sf_expert_swiglu(const void* rows, int m, int64_t row_stride,
                                int hidden_size, int intermediate_size,
                                const void* packed_weights, void* act_workspace,
                                void* out, sf_stream_t stream) {
  if (m < 0 || hidden_size < 1 || intermediate_size < 1 || row_stride < hidden_size)
    return SF_ERR_INVALID_ARGUMENT;
  if (m == 0) return SF_OK;
  if (!rows || !packed_weights || !act_workspace || !out) return SF_ERR_INVALID_ARGUMENT;
  const bool mfma = mfma_shape_ok(hidden_size, intermediate_size) && aligned16(rows) &&
                    (row_stride % 8 == 0) && aligned16(packed_weights) &&
                    aligned16(act_workspace);
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
  return launch<Resolve::kDense>(a, 1, mfma, m, reinterpret_cast<hipStream_t>(stream));
}
