// K3: grouped SwiGLU expert MLP for the verification path on gfx950.
// Restates _expert_forward and the routing-weight scale of the reference
// (src/specfit/runtime/qwen3_offloaded_experts.py:38-62, 132-138, 186-198):
//   gu  = bf16(x . GU^T), act = bf16(bf16(silu(gate)) * up),
//   y   = bf16(act . D^T), row = bf16(y * w_route)
// with GU = packed[0:2IH] as [2I, H] and D = packed[2IH:] as [H, I].
//
// At verification sizes an expert sees m <= a few dozen rows, so each weight
// element is used m times: the GEMMs are bound by streaming the 9 MiB of
// expert weights from HBM.  Both phases therefore stream every weight byte
// exactly once straight into MFMA operand registers (16-byte loads, no LDS
// round trip), with the token rows (a few KiB, L2 resident) as the other
// operand.
//
// Phase 1 (gate/up): a workgroup owns 16 activation columns of one expert,
// i.e. 16 gate rows + 16 up rows of GU (2 x 16 x H bf16).  Its 4 wavefronts
// split H into quarters; partial tiles are summed in LDS in wavefront order
// (deterministic), then the SwiGLU epilogue writes bf16 activations.
// Phase 2 (down): a workgroup owns 64 output columns (4 wavefronts x 16) of
// one expert over the full I, the epilogue applies the routing weight.
// MFMA: v_mfma_f32_16x16x32_bf16, A = token rows (M), B = weight rows (N).
#include "sf_common.h"

namespace {

constexpr int kMaxListExperts = 128;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / SF_WAVE;
constexpr int kMTiles = 4;             // 16-row MFMA tiles per pass (64 rows)
constexpr int kPassRows = 16 * kMTiles;
constexpr int kGateCols = 16;          // activation columns per phase-1 workgroup
constexpr int kDownCols = 16 * kWaves; // output columns per phase-2 workgroup
constexpr int kUnroll1 = 4;
constexpr int kUnroll2 = 8;

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

// ---------------------------------------------------------------- phase 1 --
template <Resolve R>
__global__ __launch_bounds__(kThreads) void gateup_mfma_kernel(const SwigluArgs a) {
  __shared__ float s_part[kWaves][2][kPassRows][kGateCols];
  const int tiles = a.I / kGateCols;
  const int j = blockIdx.x / tiles;
  const int tile = blockIdx.x - j * tiles;
  ExpertWork wk;
  if (!resolve<R>(a, j, wk)) return;
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int H = a.H;
  const int c0 = tile * kGateCols;
  const int kq = H / kWaves;  // this wavefront's K range
  const int kbeg = wave * kq;
  const int lrow = lane & 15;
  const int kl = 8 * (lane >> 4);
  const uint16_t* wg = wk.w + static_cast<int64_t>(c0 + lrow) * H + kbeg + kl;
  const uint16_t* wu = wk.w + static_cast<int64_t>(a.I + c0 + lrow) * H + kbeg + kl;
  const int steps = kq / 32;

  for (int p0 = 0; p0 < wk.m; p0 += kPassRows) {
    const int mp = min(kPassRows, wk.m - p0);
    const int mt_live = (mp + 15) / 16;
    const uint16_t* xr[kMTiles];
#pragma unroll
    for (int mt = 0; mt < kMTiles; ++mt) {
      const int row = mt * 16 + lrow;
      xr[mt] = row < mp ? row_ptr<R>(a, wk.r0 + p0 + row) + kbeg + kl : nullptr;
    }
    sf_f32x4 acc[kMTiles][2];
#pragma unroll
    for (int mt = 0; mt < kMTiles; ++mt) {
      acc[mt][0] = sf_f32x4{0.f, 0.f, 0.f, 0.f};
      acc[mt][1] = sf_f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int s = 0; s < steps; s += kUnroll1) {
      uint4 bg[kUnroll1], bu[kUnroll1];
#pragma unroll
      for (int u = 0; u < kUnroll1; ++u) {
        bg[u] = ld16(wg + (s + u) * 32);
        bu[u] = ld16(wu + (s + u) * 32);
      }
#pragma unroll
      for (int mt = 0; mt < kMTiles; ++mt) {
        if (mt < mt_live) {
          uint4 xa[kUnroll1];
#pragma unroll
          for (int u = 0; u < kUnroll1; ++u)
            xa[u] = xr[mt] ? ld16(xr[mt] + (s + u) * 32) : make_uint4(0, 0, 0, 0);
#pragma unroll
          for (int u = 0; u < kUnroll1; ++u) {
            acc[mt][0] = mfma16(xa[u], bg[u], acc[mt][0]);
            acc[mt][1] = mfma16(xa[u], bu[u], acc[mt][1]);
          }
        }
      }
    }
    // D layout: lane holds rows 4*(lane/16)+i, column lane%16.
#pragma unroll
    for (int mt = 0; mt < kMTiles; ++mt) {
      if (mt < mt_live) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = mt * 16 + 4 * (lane >> 4) + i;
          s_part[wave][0][row][lrow] = acc[mt][0][i];
          s_part[wave][1][row][lrow] = acc[mt][1][i];
        }
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

// ---------------------------------------------------------------- phase 2 --
template <Resolve R>
__global__ __launch_bounds__(kThreads) void down_mfma_kernel(const SwigluArgs a) {
  const int tiles = a.H / kDownCols;
  const int j = blockIdx.x / tiles;
  const int tile = blockIdx.x - j * tiles;
  ExpertWork wk;
  if (!resolve<R>(a, j, wk)) return;
  const int lane = threadIdx.x & (SF_WAVE - 1);
  const int wave = threadIdx.x / SF_WAVE;
  const int I = a.I;
  const int n0 = tile * kDownCols + wave * 16;
  const int lrow = lane & 15;
  const int kl = 8 * (lane >> 4);
  const uint16_t* wd = wk.w + 2 * static_cast<int64_t>(a.I) * a.H +
                       static_cast<int64_t>(n0 + lrow) * I + kl;
  const int steps = I / 32;

  for (int p0 = 0; p0 < wk.m; p0 += kPassRows) {
    const int mp = min(kPassRows, wk.m - p0);
    const int mt_live = (mp + 15) / 16;
    sf_f32x4 acc[kMTiles];
#pragma unroll
    for (int mt = 0; mt < kMTiles; ++mt) acc[mt] = sf_f32x4{0.f, 0.f, 0.f, 0.f};
    const uint16_t* ar[kMTiles];
#pragma unroll
    for (int mt = 0; mt < kMTiles; ++mt) {
      const int row = mt * 16 + lrow;
      ar[mt] = row < mp ? a.act + static_cast<int64_t>(wk.r0 + p0 + row) * I + kl : nullptr;
    }
    int s = 0;
    for (; s + kUnroll2 <= steps; s += kUnroll2) {
      uint4 b[kUnroll2];
#pragma unroll
      for (int u = 0; u < kUnroll2; ++u) b[u] = ld16(wd + (s + u) * 32);
#pragma unroll
      for (int mt = 0; mt < kMTiles; ++mt) {
        if (mt < mt_live) {
          uint4 xa[kUnroll2];
#pragma unroll
          for (int u = 0; u < kUnroll2; ++u)
            xa[u] = ar[mt] ? ld16(ar[mt] + (s + u) * 32) : make_uint4(0, 0, 0, 0);
#pragma unroll
          for (int u = 0; u < kUnroll2; ++u) acc[mt] = mfma16(xa[u], b[u], acc[mt]);
        }
      }
    }
    for (; s < steps; ++s) {
      const uint4 b = ld16(wd + s * 32);
#pragma unroll
      for (int mt = 0; mt < kMTiles; ++mt) {
        if (mt < mt_live) {
          const uint4 xa = ar[mt] ? ld16(ar[mt] + s * 32) : make_uint4(0, 0, 0, 0);
          acc[mt] = mfma16(xa, b, acc[mt]);
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < kMTiles; ++mt) {
      if (mt < mt_live) {
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
  return H % (kWaves * 32 * kUnroll1) == 0 && H % kDownCols == 0 &&
         I % kGateCols == 0 && I % 32 == 0;
}

template <Resolve R>
int launch(const SwigluArgs& a, int groups, bool mfma, hipStream_t s) {
  if (groups <= 0) return SF_OK;
  if (mfma) {
    const long long g1 = static_cast<long long>(groups) * (a.I / kGateCols);
    const long long g2 = static_cast<long long>(groups) * (a.H / kDownCols);
    if (g1 > 0x7fffffffLL || g2 > 0x7fffffffLL) return SF_ERR_UNSUPPORTED_SHAPE;
    gateup_mfma_kernel<R><<<dim3(static_cast<unsigned>(g1)), dim3(kThreads), 0, s>>>(a);
    SF_LAUNCH_CHECK();
    down_mfma_kernel<R><<<dim3(static_cast<unsigned>(g2)), dim3(kThreads), 0, s>>>(a);
    SF_LAUNCH_CHECK();
  } else {
    gateup_generic_kernel<R><<<dim3(groups), dim3(kThreads), 0, s>>>(a);
    SF_LAUNCH_CHECK();
    down_generic_kernel<R><<<dim3(groups), dim3(kThreads), 0, s>>>(a);
    SF_LAUNCH_CHECK();
  }
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
                                 int intermediate_size, int n_experts,
                                 const int32_t* expert_ids,
                                 const uint64_t* expert_weights,
                                 void* act_workspace, void* out_rows,
                                 sf_stream_t stream) {
  int rc = check_common(tokens, top_k, hidden_size, intermediate_size);
  if (rc) return rc;
  if (n_experts < 0) return SF_ERR_INVALID_ARGUMENT;
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
    rc = launch<Resolve::kList>(a, a.n, mfma, s);
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
  return launch<Resolve::kTable>(a, num_experts, mfma, reinterpret_cast<hipStream_t>(stream));
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
  return launch<Resolve::kDense>(a, 1, mfma, reinterpret_cast<hipStream_t>(stream));
}
