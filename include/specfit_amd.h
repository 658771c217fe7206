/*
 * specfit_amd.h -- C ABI of the MI355X (gfx950) offloaded Qwen3-MoE
 * verification path.
 *
 * Every entry point is enqueue-only: it validates its arguments on the host,
 * launches HIP work on the caller's stream and returns.  Nothing here
 * allocates device memory, synchronises the host, or keeps mutable global
 * state; all buffers are owned by the caller.  Return value 0 means success;
 * a non-zero value is an SF_ERR_* code (argument errors) or a hipError_t
 * offset by SF_ERR_HIP_BASE.  sf_error_string() names either kind.
 *
 * Data types: "bf16" buffers hold IEEE bfloat16 bit patterns (uint16_t);
 * integer buffers are little-endian.  Streams are hipStream_t passed as an
 * opaque pointer (NULL = the legacy default stream).
 *
 * Reference interfaces replaced (paths relative to the SpecFit tree; "tf:" is
 * transformers/models/qwen3_moe/modeling_qwen3_moe.py of the pinned
 * transformers release):
 *   sf_router_topk       tf:258-267  Qwen3MoeTopKRouter.forward
 *   sf_dispatch          src/specfit/runtime/qwen3_offloaded_experts.py:173-178
 *                        (stable sort + unique_consecutive + route_tokens) and
 *                        :111-113,120-122 (unique / where of the legacy path)
 *   sf_grouped_swiglu    qwen3_offloaded_experts.py:38-62 (_expert_forward),
 *                        :132-138 and :198 (routing-weight scale), :186-190
 *                        (route gather)
 *   sf_expert_swiglu     qwen3_offloaded_experts.py:38-62 (_expert_forward
 *                        on already-gathered rows, no weight scale)
 *   sf_combine           qwen3_offloaded_experts.py:144-164 and :200-202
 *                        (index_add_ in canonical or arrival order)
 *   sf_copy_h2d          src/specfit/runtime/gpu_expert_cache.py:556-561
 *                        (slot.tensor.copy_(pinned_source, non_blocking=True))
 *   sf_expert_decode     the same copy when the transfer moves an
 *                        exponent-coded record (decoded into the slot)
 *   sf_tree_attention    the attention of the verification forward:
 *                        eagle3_tree.py:1202-1240 runs the target with
 *                        Eagle3DraftTree.verification_attention_mask
 *                        (eagle3_types.py:450-473); each Qwen3 attention layer
 *                        then calls transformers sdpa_attention_forward
 *                        (integrations/sdpa_attention.py) with that mask
 *   sf_rms_norm          tf:294-299  Qwen3MoeRMSNorm.forward (the four norms
 *                        of every decoder layer of the verification forward)
 *   sf_qk_norm_rope      tf:162-167  the query/key norms and
 *                        apply_rotary_pos_emb (tf:58-81) of
 *                        Qwen3MoeAttention.forward
 */
#ifndef SPECFIT_AMD_H
#define SPECFIT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SF_ABI_VERSION 13

/* Argument error codes (hipError_t values are returned as SF_ERR_HIP_BASE + e). */
#define SF_OK 0
#define SF_ERR_INVALID_ARGUMENT 1
#define SF_ERR_UNSUPPORTED_SHAPE 2
#define SF_ERR_MISALIGNED 3
#define SF_ERR_TOO_MANY_EXPERTS 4
#define SF_ERR_SCRATCH_LIMIT 5
#define SF_ERR_HIP_BASE 1000

/* Largest expert count the router, dispatch and combine kernels accept. */
#define SF_MAX_EXPERTS 256
/* Largest top-k. */
#define SF_MAX_TOPK 32
/* Values per chunk of an exponent-coded expert record (sf_expert_decode). */
#define SF_DECODE_CHUNK 4096

typedef void *sf_stream_t;

/* ABI version of the loaded library (SF_ABI_VERSION at build time). */
int sf_abi_version(void);

/* Static description of an error code; never NULL. */
const char *sf_error_string(int code);

/*
 * K1: router.  Replaces Qwen3MoeTopKRouter.forward (tf:258-267).
 *   logits[t,e] = bf16( sum_k hidden[t,k] * router_weight[e,k] )   (fp32 sum)
 *   p[t,:]      = softmax_fp32(logits[t,:])
 *   (v, idx)    = top_k(p[t,:]) in descending p; equal p -> lower expert id
 *   w[t,j]      = bf16( v_j / (v_0 + ... + v_{k-1}) )   if norm_topk_prob
 *               = bf16( v_j )                          otherwise
 * The fp32 summation order of the dot product and of the softmax sum is
 * fixed (see the kernel source), so logits, weights and indices are a pure
 * function of the inputs.
 *   hidden        bf16 [tokens, hidden_size]
 *   router_weight bf16 [num_experts, hidden_size]
 *   logits        bf16 [tokens, num_experts]          (output)
 *   topk_weights  bf16 [tokens, top_k]                (output)
 *   topk_index    int64 [tokens, top_k]               (output)
 * Limits: 1 <= num_experts <= SF_MAX_EXPERTS, 1 <= top_k <= min(num_experts,
 * SF_MAX_TOPK), hidden_size >= 1.  tokens == 0 launches nothing.
 */
int sf_router_topk(const void *hidden, const void *router_weight, int tokens,
                   int hidden_size, int num_experts, int top_k,
                   int norm_topk_prob, void *logits, void *topk_weights,
                   int64_t *topk_index, sf_stream_t stream);

/*
 * K2: token-to-expert dispatch.  Replaces the stable sort of the flattened
 * routes by expert id (qwen3_offloaded_experts.py:173-178).
 *   topk_index int64 [tokens, top_k]
 *   counts     int32 [num_experts + 1]  routes per expert; counts[num_experts]
 *              = number of entries outside [0, num_experts) (not dispatched)
 *   offsets    int32 [num_experts + 1]  exclusive prefix sum of counts
 *   perm_pos   int32 [tokens * top_k]   route position (t * top_k + j) of each
 *              permuted row; rows of one expert are contiguous and keep
 *              ascending position order (stable)
 *   inv_perm   int32 [tokens * top_k]   permuted row of each route position
 *              (-1 for an out-of-range entry)
 *   host_meta  NULL, or pinned host memory (hipHostMalloc) of int32
 *              [2, num_experts + 1]: the kernel also writes counts (row 0)
 *              and offsets (row 1) there, so the caller reads the routes per
 *              expert once the stream passes the kernel, with no separate
 *              device-to-host copy (the reference's one host read of the
 *              routed experts, qwen3_offloaded_experts.py:111-113).  Memory
 *              the device cannot map returns SF_ERR_INVALID_ARGUMENT.
 * One workgroup; any tokens >= 0.
 */
int sf_dispatch(const int64_t *topk_index, int tokens, int top_k,
                int num_experts, int32_t *counts, int32_t *offsets,
                int32_t *perm_pos, int32_t *inv_perm, int32_t *host_meta,
                sf_stream_t stream);

/*
 * K3: grouped SwiGLU expert MLP over dispatched rows.  Replaces the per-expert
 * loop of _expert_forward + weight scale (qwen3_offloaded_experts.py:38-62,
 * 132-138, 186-198).  For each listed expert e with rows
 * r in [offsets[e], offsets[e+1]) and token t = perm_pos[r] / top_k:
 *   gu   = bf16(hidden[t] . GU^T)          GU = packed[0 : 2*I*H] as [2I, H]
 *   act  = bf16(bf16(silu(gu[:I])) * gu[I:])
 *   y    = bf16(act . D^T)                 D  = packed[2*I*H :] as [H, I]
 *   rows[r] = bf16(y * route_weights[perm_pos[r]])   (y if route_weights NULL)
 * Packed expert layout: [gate (I x H) | up (I x H) | down (H x I)], row-major
 * bf16, as written by the reference's packed checkpoint.
 *   max_rows        an upper bound on the rows of any listed expert
 *                   (tokens * top_k always is).  It picks the kernel build
 *                   (registers sized for that many rows).  Any value >= 1
 *                   computes every row; with a value below some expert's
 *                   row count that expert's fp32 summation order is the one
 *                   of a smaller expert.
 * The MFMA kernels cover the Qwen3-30B-A3B (hidden 2048, intermediate 768)
 * and Qwen3-235B-A22B (hidden 4096, intermediate 1536) expert shapes with
 * 16-byte aligned buffers; other shapes run fp32 loop kernels with the same
 * rounding points.  The fp32 summation order of
 * an output depends on the shape and on its expert's row count only.
 *   expert_ids      host int32 [n_experts]: experts computed by this call
 *   expert_weights  host uint64 [n_experts]: device address of each expert's
 *                   packed weights (a cache slot)
 *   expert_row_begin, expert_row_count
 *                   host int32 [n_experts] each, or both NULL: each listed
 *                   expert's first permuted row and row count
 *                   (offsets[e] and offsets[e+1] - offsets[e]).  A caller
 *                   that has read the dispatch counts passes them, so the
 *                   kernels start streaming weights without first reading
 *                   offsets from device memory; with NULL they read them.
 *   act_workspace   bf16 [tokens * top_k, intermediate_size] scratch
 *   out_rows        bf16 [tokens * top_k, hidden_size] (rows of listed
 *                   experts are written, others untouched)
 * Experts of one call are independent; the result of an expert does not
 * depend on which other experts share the call.
 */
int sf_grouped_swiglu(const void *hidden, const int32_t *perm_pos,
                      const int32_t *offsets, const void *route_weights,
                      int tokens, int top_k, int hidden_size,
                      int intermediate_size, int n_experts, int max_rows,
                      const int32_t *expert_ids,
                      const uint64_t *expert_weights,
                      const int32_t *expert_row_begin,
                      const int32_t *expert_row_count, void *act_workspace,
                      void *out_rows, sf_stream_t stream);

/*
 * K3, device slot-table form: computes every expert e < num_experts whose
 * slot_of_expert[e] >= 0 and that has at least one row, reading its weights
 * at slot_base + slot_of_expert[e] * slot_stride_elems (bf16 elements).
 * slot_of_expert is a device int32 [num_experts] array whose entries are -1
 * or the index of a slot behind slot_base (the kernel trusts them, as it
 * trusts slot_base itself).  Needs no host-side knowledge of which experts
 * are active (no device-to-host read).
 * max_rows bounds the rows of any expert as for sf_grouped_swiglu (tokens
 * is one when every token's top_k experts are distinct, as a router's are).
 */
int sf_grouped_swiglu_table(const void *hidden, const int32_t *perm_pos,
                            const int32_t *offsets, const void *route_weights,
                            int tokens, int top_k, int hidden_size,
                            int intermediate_size, int num_experts, int max_rows,
                            const int32_t *slot_of_expert,
                            const void *slot_base, int64_t slot_stride_elems,
                            void *act_workspace, void *out_rows,
                            sf_stream_t stream);

/*
 * K3, device slot-table form, allocating nothing.  No counterpart in the
 * reference: this entry point is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, results and limits as
 * sf_grouped_swiglu_table minus act_workspace: the [tokens * top_k,
 * intermediate_size] bf16 activation workspace is taken from a fixed device
 * array of SF_NOALLOC_SCRATCH_BYTES that each GPU the library runs on holds
 * until the process ends.
 * Limit: tokens * top_k * intermediate_size * 2 <= SF_NOALLOC_SCRATCH_BYTES
 * (4 MiB: 341 tokens at top_k 8 and intermediate 768), else
 * SF_ERR_SCRATCH_LIMIT and nothing is launched.
 * Every call on one GPU shares that GPU's array, which keeps the last
 * call's contents: calls that overlap on one GPU (kernels on concurrent
 * streams, or host threads) race.  Nothing in it needs to start at zero:
 * each activation row a launch reads is written first by the same launch.
 */
#define SF_NOALLOC_SCRATCH_BYTES (4u << 20)
int sf_grouped_swiglu_table_noalloc(const void *hidden, const int32_t *perm_pos,
                                    const int32_t *offsets,
                                    const void *route_weights, int tokens,
                                    int top_k, int hidden_size,
                                    int intermediate_size, int num_experts,
                                    int max_rows,
                                    const int32_t *slot_of_expert,
                                    const void *slot_base,
                                    int64_t slot_stride_elems, void *out_rows,
                                    sf_stream_t stream);

/*
 * K3 on already-gathered rows of one expert (the _expert_forward seam,
 * qwen3_offloaded_experts.py:38-62): out[m, H] = y without weight scale.
 *   rows bf16 [m, hidden_size] (row stride row_stride elements)
 */
int sf_expert_swiglu(const void *rows, int m, int64_t row_stride,
                     int hidden_size, int intermediate_size,
                     const void *packed_weights, void *act_workspace,
                     void *out, sf_stream_t stream);

/*
 * K4: weighted combine.  Replaces zeros_like + index_add_ of the expert
 * contributions (qwen3_offloaded_experts.py:144-164, 200-202).
 *   out[t] = sum over the routes j of token t, in ascending
 *            (expert_rank[topk_index[t,j]], j) order, of rows[inv_perm[t*K+j]]
 * With accumulate_fp32 == 0 every addition rounds to bf16, exactly as
 * sequential bf16 index_add_ calls; otherwise the sum is fp32 and rounded once.
 *   rows         bf16 [tokens * top_k, hidden_size] (K3 output)
 *   expert_rank  host int32 [num_experts] execution rank of each expert, or
 *                NULL for canonical ascending expert id
 *   out          bf16 [tokens, hidden_size]
 */
int sf_combine(const void *rows, const int64_t *topk_index,
               const int32_t *inv_perm, const int32_t *expert_rank,
               int tokens, int top_k, int num_experts, int hidden_size,
               int accumulate_fp32, void *out, sf_stream_t stream);

/*
 * Host-to-device copy of an expert from pinned (page-locked) host memory into
 * a cache slot, enqueued on `stream` (SDMA).  Replaces the non-blocking
 * slot.tensor.copy_(pinned) of gpu_expert_cache.py:556-561.
 */
int sf_copy_h2d(void *device_dst, const void *host_src, size_t bytes,
                sf_stream_t stream);

/*
 * Exponent-coded expert records: the host-to-device transfer of an expert
 * may move a lossless record of its bf16 weights instead of the raw bytes
 * (about 67% of them for N(0, 0.02) weights), decoded into the slot on the
 * device.  Together with sf_copy_h2d of the record into a staging buffer
 * this replaces the same slot.tensor.copy_(pinned_source)
 * (gpu_expert_cache.py:556-561); the slot ends with the same bytes.  The
 * exponent of a value is a cascade of codes into the 32-byte table:
 *   level 1, 2 bits (every value):       c < 3: table[c];       3: level 2
 *   level 2, 2 bits (n2 values):         c < 3: table[8 + c];   3: level 3
 *   level 3, 4 bits (n3 values):         c < 15: table[16 + c]; 15: raw byte
 * Record of n values (every section 256-byte aligned):
 *   S   [n] uint8                 sign << 7 | mantissa of value i
 *   P   2 planes of ceil(n/16) uint16 words: bit i%16 of word i/16 of
 *                                 plane p is bit p of value i's level-1 code
 *   L2  [ceil(n2/4)] uint8        level-2 codes in value order, entry j at
 *                                 bits 2(j%4) of byte j/4
 *   L3  [ceil(n3/2)] uint8        level-3 codes in value order, entry j at
 *                                 bits 4(j%2) of byte j/2
 *   R   [nr] uint8                raw exponent bytes in value order
 *   C2, C3, CR [c + 1] uint32     L2, L3 and R entries of the values before
 *                                 value k * SF_DECODE_CHUNK
 *                                 (c = ceil(n / SF_DECODE_CHUNK))
 * sf_expert_record_bytes returns the record size (-1 for invalid counts;
 * valid: 0 <= n_raw <= n_third <= n_second <= n_values).
 * sf_expert_decode writes out[i] = sign | exponent | mantissa of value i:
 *   record          device buffer of at least record_bytes >= the record size
 *   exponent_table  host array of 32 exponent bytes (entries 3..7, 11..15
 *                   and 31 unused)
 *   out             bf16 [n_values], 16-byte aligned like record
 */
int64_t sf_expert_record_bytes(int64_t n_values, int64_t n_second, int64_t n_third,
                               int64_t n_raw);
int sf_expert_decode(const void *record, size_t record_bytes, int64_t n_values,
                     const uint8_t *exponent_table, int n_second, int n_third, int n_raw,
                     void *out, sf_stream_t stream);

/*
 * K5: grouped-query attention of the verification forward over the cached
 * prefix plus the draft tree.  For query token qi and query head
 * qh = h * G + j (G = q_heads / kv_heads, h the key/value head):
 *   out[qi, qh, :] = sum_s p_s * v[h, s, :],
 *   p = softmax over admitted keys s of scale * (q[qi, qh, :] . k[h, s, :])
 * computed in fp32 and rounded to bf16 once.  Key s is admitted when
 * mask[qi * mask_stride_query + s] != 0; with mask == NULL, when
 * s <= keys - queries + qi (causal, aligned to the end of the keys).  A
 * query with no admitted key gets zeros.
 *   q     bf16, element (qi, qh, d) at qi*q_stride_token + qh*q_stride_head + d
 *   k, v  bf16, element (h, s, d) at h*stride_head + s*stride_token + d
 *         (k: 16-byte aligned rows)
 *   mask  uint8/bool [queries, >= keys] with row stride mask_stride_query
 *   out   bf16 [queries, q_heads, head_dim], contiguous
 * head_dim % 8 == 0, head_dim <= 256, G in {1, 2, 4, 8, 16}.
 */
int sf_tree_attention(const void *q, int64_t q_stride_token,
                      int64_t q_stride_head, const void *k,
                      int64_t k_stride_head, int64_t k_stride_token,
                      const void *v, int64_t v_stride_head,
                      int64_t v_stride_token, const uint8_t *mask,
                      int64_t mask_stride_query, int queries, int keys,
                      int q_heads, int kv_heads, int head_dim, float scale,
                      void *out, sf_stream_t stream);

/*
 * K6: RMSNorm over the last dimension.  Replaces Qwen3MoeRMSNorm.forward
 * (tf:294-299):
 *   v = mean over d of float(x[r, d])^2 (fp32)
 *   out[r, d] = bf16(float(weight[d]) * bf16(float(x[r, d]) * rsqrt(v + eps)))
 *   x       bf16, row r at x + r * row_stride (elements), dim elements
 *   weight  bf16 [dim]
 *   out     bf16, row r at out + r * out_stride (may equal x: in place)
 * The fp32 sum of squares runs in a fixed order of its own, so results can
 * differ from the eager module by a last-place rounding of the variance.
 */
int sf_rms_norm(const void *x, int64_t row_stride, int rows, int dim,
                const void *weight, float eps, void *out, int64_t out_stride,
                sf_stream_t stream);

/*
 * K7: query/key RMSNorm and rotary embedding of one attention layer (batch
 * 1).  Replaces, in Qwen3MoeAttention.forward (tf:162-167),
 * q_norm(q.view(T, Hq, D)), k_norm(k.view(T, Hk, D)) and
 * apply_rotary_pos_emb (tf:58-81):
 *   n = sf_rms_norm's row result (same bits)
 *   out[h, t, d] = bf16(bf16(n[d] * cos[t, d]) + bf16(rot(n)[d] * sin[t, d]))
 *   rot(n)[d] = -n[d + D/2] for d < D/2, n[d - D/2] otherwise
 *   q, k        bf16 [tokens, q_heads | kv_heads, head_dim]: token t at
 *               q + t * q_stride_token (elements; >= q_heads * head_dim and a
 *               multiple of 8, e.g. one fused q/k/v projection row), heads
 *               contiguous within a token
 *   q_weight, k_weight  bf16 [head_dim]
 *   cos, sin    bf16 [tokens, head_dim], contiguous
 *   q_out, k_out  bf16 [q_heads | kv_heads, tokens, head_dim], contiguous
 * head_dim must be 128 (SF_ERR_UNSUPPORTED_SHAPE otherwise); all buffers
 * 16-byte aligned.
 */
int sf_qk_norm_rope(const void *q, int64_t q_stride_token, const void *k,
                    int64_t k_stride_token, int tokens, int q_heads,
                    int kv_heads, int head_dim, const void *q_weight,
                    const void *k_weight, float eps, const void *cos,
                    const void *sin, void *q_out, void *k_out,
                    sf_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SPECFIT_AMD_H */
