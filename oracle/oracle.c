/*
 * CPU oracle for the offloaded Qwen3-MoE verification path -- TEST
 * INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only to check results (or as
 * the timed CPU baseline); the product path never calls it.
 *
 * Bit-exact restatement of the integer/byte parts and of the router:
 *   oracle_router    tf:258-267 (Qwen3MoeTopKRouter.forward), with the fp32
 *                    summation order and exp() that the GPU kernel fixes
 *   oracle_dispatch  src/specfit/runtime/qwen3_offloaded_experts.py:173-178
 *                    (stable sort of the flattened routes by expert id)
 *   oracle_combine   qwen3_offloaded_experts.py:144-164, 200-202
 *                    (zeros_like + index_add_ in canonical / arrival order)
 * Build with -ffp-contract=off: every fused multiply-add below is explicit.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define WAVE 64

static float bf16_to_f32(uint16_t v) {
  uint32_t u = (uint32_t)v << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

/* exp(x) for x <= 0: Cody-Waite reduction + degree-7 Taylor polynomial (the
 * textbook method), zero below 2^-126. */
float oracle_exp_nonpos(float x) {
  if (!(x > -87.0f)) return 0.0f;
  float n = rintf(x * 1.44269504088896341f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.42860682030941723e-06f, r);
  float p = 1.98412698412698413e-04f;
  p = fmaf(p, r, 1.38888888888888889e-03f);
  p = fmaf(p, r, 8.33333333333333333e-03f);
  p = fmaf(p, r, 4.16666666666666667e-02f);
  p = fmaf(p, r, 1.66666666666666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni <= -126) return 0.0f;
  uint32_t bits = (uint32_t)(ni + 127) << 23;
  float scale;
  memcpy(&scale, &bits, 4);
  return p * scale;
}

/* Combine 64 lane partials with the xor butterfly d = 1, 2, ..., 32 and
 * return the (lane-invariant) result. */
static float butterfly_sum(float *v) {
  float next[WAVE];
  for (int d = 1; d <= 32; d <<= 1) {
    for (int l = 0; l < WAVE; ++l) next[l] = v[l] + v[l ^ d];
    memcpy(v, next, sizeof(next));
  }
  return v[0];
}

/* One router logit: lane l owns chunks c = l + 64 i of 8 elements and sums in
 * ascending k; lanes are combined by the butterfly. */
static float router_dot(const uint16_t *h, const uint16_t *w, int H) {
  float part[WAVE];
  int nchunks = (H + 7) / 8;
  for (int l = 0; l < WAVE; ++l) {
    float acc = 0.0f;
    for (int c = l; c < nchunks; c += WAVE)
      for (int j = 0; j < 8; ++j) {
        int k = c * 8 + j;
        if (k < H) acc = fmaf(bf16_to_f32(h[k]), bf16_to_f32(w[k]), acc);
      }
    part[l] = acc;
  }
  return butterfly_sum(part);
}

void oracle_router(const uint16_t *hidden, const uint16_t *wr, int T, int H,
                   int E, int K, int renorm, uint16_t *logits, uint16_t *topw,
                   int64_t *topi, float *probs /* [T,E] or NULL */) {
  float lg[256], x[256], p[256];
  int live[256];
  for (int t = 0; t < T; ++t) {
    const uint16_t *h = hidden + (size_t)t * H;
    for (int e = 0; e < E; ++e) {
      uint16_t b = f32_to_bf16(router_dot(h, wr + (size_t)e * H, H));
      logits[(size_t)t * E + e] = b;
      lg[e] = bf16_to_f32(b);
    }
    float m = -INFINITY;
    for (int e = 0; e < E; ++e) m = fmaxf(m, lg[e]);
    float part[WAVE];
    for (int l = 0; l < WAVE; ++l) {
      float s = 0.0f;
      for (int e = l; e < E; e += WAVE) {
        x[e] = oracle_exp_nonpos(lg[e] - m);
        s += x[e];
      }
      part[l] = s;
    }
    float total = butterfly_sum(part);
    for (int e = 0; e < E; ++e) {
      p[e] = x[e] / total;
      live[e] = 1;
      if (probs) probs[(size_t)t * E + e] = p[e];
    }
    float val[32];
    int id[32];
    for (int r = 0; r < K; ++r) {
      int best = -1;
      for (int e = 0; e < E; ++e)
        if (live[e] && (best < 0 || p[e] > p[best])) best = e;
      live[best] = 0;
      val[r] = p[best];
      id[r] = best;
    }
    float sum = 0.0f;
    for (int r = 0; r < K; ++r) sum += val[r];
    for (int r = 0; r < K; ++r) {
      float v = renorm ? val[r] / sum : val[r];
      topw[(size_t)t * K + r] = f32_to_bf16(v);
      topi[(size_t)t * K + r] = id[r];
    }
  }
}

/* Stable counting sort of route positions by expert id. */
void oracle_dispatch(const int64_t *idx, int T, int K, int E, int32_t *counts,
                     int32_t *offsets, int32_t *perm_pos, int32_t *inv_perm) {
  int n = T * K;
  int invalid = 0;
  for (int e = 0; e <= E; ++e) counts[e] = 0;
  for (int i = 0; i < n; ++i) {
    if (idx[i] >= 0 && idx[i] < E)
      counts[idx[i]]++;
    else
      invalid++;
  }
  int run = 0;
  for (int e = 0; e < E; ++e) {
    offsets[e] = run;
    run += counts[e];
  }
  offsets[E] = run;
  counts[E] = invalid;
  int32_t fill[257];
  for (int e = 0; e < E; ++e) fill[e] = offsets[e];
  for (int i = 0; i < n; ++i) {
    if (idx[i] >= 0 && idx[i] < E) {
      int pos = fill[idx[i]]++;
      perm_pos[pos] = i;
      inv_perm[i] = pos;
    } else {
      inv_perm[i] = -1;
    }
  }
}

/* out[t] = sum of rows of token t's routes in (rank, position) order; each
 * addition rounded to bf16 unless acc_fp32. */
void oracle_combine(const uint16_t *rows, const int64_t *idx,
                    const int32_t *inv_perm, const int32_t *rank /* or NULL */,
                    int T, int K, int E, int H, int acc_fp32, uint16_t *out) {
  int order[64];
  int keys[64];
  for (int t = 0; t < T; ++t) {
    int n = 0;
    for (int j = 0; j < K; ++j) {
      int64_t e = idx[(size_t)t * K + j];
      int r = inv_perm[(size_t)t * K + j];
      if (e < 0 || e >= E || r < 0) continue;
      int key = rank ? rank[e] : (int)e;
      int p = n++;
      while (p > 0 && keys[p - 1] > key) {
        keys[p] = keys[p - 1];
        order[p] = order[p - 1];
        --p;
      }
      keys[p] = key;
      order[p] = r;
    }
    for (int c = 0; c < H; ++c) {
      float acc = 0.0f;
      for (int q = 0; q < n; ++q) {
        float s = acc + bf16_to_f32(rows[(size_t)order[q] * H + c]);
        acc = acc_fp32 ? s : round_bf16(s);
      }
      out[(size_t)t * H + c] = f32_to_bf16(acc);
    }
  }
}
