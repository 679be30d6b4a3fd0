/* flashgrpo_amd: C ABI of the MI355X (gfx950) speculative-rollout kernels.
 *
 * Every entry point is stream-ordered and asynchronous: device pointers in,
 * device pointers out, `stream` is a hipStream_t (torch's current stream when
 * called from Python). Nothing here allocates device memory; scratch space is a
 * caller-provided `workspace`. Return value: 0 on success, <0 on error, with a
 * message from fg_last_error() (thread-local). Shapes are validated on the host
 * before any launch; index data that only exists on the device is bounds-checked
 * in the kernel and reported through an `err_flag` word (0 = ok).
 *
 * dtype codes: 0 = fp32, 1 = bf16. Token ids and indices are int32.
 *
 * Reference interfaces replaced (ihbkaiser/ss-GRPO, flashgrpo/):
 *   fg_medusa_heads     models/medusa_heads.py:74-78 (project_hidden),
 *                       decoding/flash_medusa_decoder.py:254-294
 *   fg_lm_head          decoding/flash_medusa_decoder.py:289-294, 414-433, 1079-1091
 *   fg_medusa_topk      decoding/medusa_tree.py:239-252 (per-depth torch.topk),
 *                       decoding/flash_medusa_decoder.py:320-339 (confidences)
 *   fg_tree_layout      decoding/medusa_tree.py:254-277 (BFS token assembly)
 *   fg_sparse_tree_layout  flashgrpo_b200/decoding/medusa_tree.py:509-685
 *                       (_select_sparse_children + _build_sparse_batch_trees)
 *   fg_rope_kv_write    models/qwen_flashgrpo_wrapper.py:172-180 (HF rotary + DynamicCache.update)
 *   fg_tree_attention   decoding/tree_attention.py:6-67 + the HF attention it feeds
 *   fg_rmsnorm, fg_swiglu  models/qwen_flashgrpo_wrapper.py:172-180 (HF decoder layer)
 *   fg_gate_up_swiglu   models/qwen_flashgrpo_wrapper.py:172-180 (the HF decoder layer's MLP
 *                       act_fn(gate_proj(x)) * up_proj(x), the two projections and the product in one GEMM)
 *   fg_linear_parts, fg_residual_rmsnorm_parts, fg_rope_kv_write_parts, fg_linear_rope_kv_write,
 *   fg_rope_cos_sin
 *                       models/qwen_flashgrpo_wrapper.py:172-180 (the HF decoder layer's q/k/v, o and
 *                       down projections, finished with the bias + rotary + cache write or the
 *                       residual add + next RMSNorm)
 *   fg_chain_cell_norm  models/medusa_heads.py:12-42 (ChainDraftCell state_norm / token_norm,
 *                       the two LayerNorms whose outputs its projections take side by side)
 *   fg_sample_tokens    decoding/acceptance.py:34-130 (sample_from_logits)
 *   fg_accept_walk      decoding/acceptance.py:179-260 (exact_accept_paths_batch);
 *   fg_walk_begin/rows/step  the same walk, one step per call (lazy LM-head rows);
 *                       flashgrpo_b200/decoding/acceptance.py:184-267 (correction tokens)
 *   fg_accept_finalize  decoding/flash_medusa_decoder.py:899-922;
 *                       flashgrpo_b200/decoding/flash_medusa_decoder.py:2303-2319
 *   fg_kv_path_gather   decoding/kv_extraction.py:87-218 (extract_accepted_path_kv)
 */
#ifndef FLASHGRPO_AMD_H
#define FLASHGRPO_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Last error message of the calling thread ("" if none). */
const char* fg_last_error(void);
int fg_version(void);

/* Medusa residual block for `heads` heads:
 *   out[h*batch + b, :] = hidden[b] + SiLU(fc_w[h] . LayerNorm_h(hidden[b]) + fc_b[h])
 * hidden [batch, H] (row stride ldh), ln_w/ln_b [heads, H] fp32, fc_w [heads, H, H],
 * fc_b [heads, H] in `dtype`; out [heads*batch, H] in out_dtype.
 * workspace >= fg_medusa_heads_workspace(batch, H, heads, dtype) bytes. */
size_t fg_medusa_heads_workspace(int batch, int hidden, int heads, int dtype);
int fg_medusa_heads(const void* hidden, int dtype, int batch, int H, int64_t ldh, int heads, const float* ln_w,
                    const float* ln_b, float ln_eps, const void* fc_w, const void* fc_b, void* out, int out_dtype,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Tied LM-head projection: out[m, :] = x[row_index ? row_index[m] : m, :] . w^T
 * x [*, K] (row stride ldx), w [N, K] (row stride ldw), out [M, N] (row stride ldo).
 * row_active (optional, [M]): output tiles whose rows are all 0 there are not computed.
 * bf16 requires K % 64 == 0 and 16-byte aligned rows. */
int fg_lm_head(const void* x, int dtype, int M, int K, int64_t ldx, const int32_t* row_index,
               const int32_t* row_active, const void* w, int64_t ldw, int N, void* out, int out_dtype, int64_t ldo,
               void* stream);

/* Tied LM head over 1..256 rows with the per-row top-k fused:
 *   logits[m, :] = x[row_index ? row_index[m] : m, :] . w^T        (bf16 x and w)
 * One persistent launch streams w [N, K] once (bf16, 16-byte aligned rows, K % 64 == 0,
 * w spanning < 4 GiB; x spanning < 4 GiB from its base); out [M, ldo] (bf16 or fp32,
 * optional). With kmax in [1, 16] (at most 8 above 192 rows) it also writes each row's top-kmax candidates
 * (cand_tokens / cand_scores [M, kmax]) and, if row_stats is given, its (max, logsumexp)
 * [M, 2], ranked and computed exactly as fg_medusa_topk does on the bf16 logits (sanitize
 * as there), without reading the logits back; workspace >=
 * fg_lm_head_topk_workspace(M, N, kmax). row_active (kmax 0 only): nothing is computed
 * when every flag is 0, and rows whose flag is 0 are not written. part_max / part_key (optional; kmax 0 with out): each workgroup
 * writes, for every row m, the maximum of the row's stored logits over its columns (NaN
 * ignored) to part_max[m * P + p] and their largest rank key (value desc, index asc,
 * NaN first: the first maximum) to part_key[m * P + p], P = fg_lm_head_topk_parts(N):
 * the row maxima fg_walk_step needs before it can weigh the logits.
 * Replaces decoding/flash_medusa_decoder.py:289-294 (Medusa rows),
 * :1079-1091 (leaf / next-round rows) and the torch.topk of medusa_tree.py:239-252. */
size_t fg_lm_head_topk_workspace(int rows, int vocab, int kmax);
int fg_lm_head_topk_parts(int vocab);
int fg_lm_head_topk(const void* x, int M, int K, int64_t ldx, const int32_t* row_index, const int32_t* row_active,
                    const void* w, int64_t ldw, int N, void* out, int out_dtype, int64_t ldo, int kmax, int sanitize,
                    int32_t* cand_tokens, float* cand_scores, float* row_stats, float* part_max, uint64_t* part_key,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Per-row top-kmax candidates, ranked (value desc, index asc).
 * logits [rows, vocab] with row stride row_stride (multiple of 8, 32-byte aligned base).
 * cand_tokens/cand_scores [rows, kmax]; row_stats (optional) [rows, 2] = (max, logsumexp).
 * sanitize != 0 ranks (and scores) nan_to_num(x, nan=-1e9, posinf=1e9, neginf=-1e9), the
 * chain builder's logits (decoding/flash_medusa_decoder.py:477-482); 0 ranks NaN first,
 * as torch.topk does (the Medusa path, decoding/medusa_tree.py:239-252).
 * workspace >= fg_medusa_topk_workspace(rows, vocab, kmax). */
size_t fg_medusa_topk_workspace(int rows, int vocab, int kmax);
int fg_medusa_topk(const void* logits, int dtype, int64_t row_stride, int rows, int vocab, int kmax, int sanitize,
                   int32_t* cand_tokens, float* cand_scores, float* row_stats, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Dense-tree tokens: tree_tokens[b, 0] = roots[b]; for n >= 1
 * tree_tokens[b, n] = cand_tokens[(node_depth[n]-2)*batch + b, node_rank[n]].
 * node_depth/node_rank [num_nodes] describe the plan's BFS topology. */
int fg_tree_layout(const int32_t* cand_tokens, const float* cand_scores, int kstride, int batch,
                   const int32_t* roots, const int32_t* node_depth, const int32_t* node_rank, int num_nodes,
                   int32_t* tree_tokens, float* tree_scores, int out_stride, void* stream);

/* Sparse asymmetric trees, one per sequence. cand_tokens/cand_scores are the
 * top-kstride lists of heads 1..heads (row h*batch + b, as fg_medusa_topk writes
 * them); nodes_by_head [heads] (host) are the per-head node counts; heads beyond
 * the third are ignored. Node order: root, head-1 nodes, greedily picked head-2
 * then head-3 (parent, candidate) pairs, leftover head-1 candidates; cut at
 * `budget`. Candidate score = value / temperature (fp32); pair value =
 * parent score + candidate score - diversity_penalty * (picks of the parent) in
 * fp64. head3_gate [batch] u8 (NULL = all rows) switches head 3 off per row, its
 * nodes then go to head 2. Outputs [batch, num_nodes] (num_nodes <= 64): tokens,
 * parents (-1 root/padding), depth (root 1, padding 0), pos_offset (depth - 1,
 * padding 0), anc (ancestor-or-self bits; padding: self), n_children, scores (fp64
 * path scores, root 0; may be NULL); n_nodes [batch]. */
int fg_sparse_tree_layout(const int32_t* cand_tokens, const float* cand_scores, int kstride, int batch,
                          int vocab, const int32_t* roots, const uint8_t* head3_gate, const int32_t* nodes_by_head,
                          int heads, int budget, float temperature, double diversity_penalty, int num_nodes,
                          int32_t* tree_tokens, int32_t* parents, int32_t* depth, int32_t* pos_offset,
                          uint64_t* anc, int32_t* n_children, int32_t* n_nodes, double* scores, void* stream);

/* Rotary embedding of q and k for num_nodes new tokens per sequence, and the
 * K/V write into cache slots seq_len[b] + n. qkv [batch*num_nodes, (Hq+2Hkv)*d]
 * (row stride ld_qkv); position = seq_len[b] + pos_offset[b*pos_batch_stride + n]
 * (stride 0: one offset list for every sequence); inv_freq [d/2] fp32;
 * q_out [batch, num_nodes, Hq, d]; caches [Bc, Hkv, capacity, d]; row_map maps b to
 * its cache row (NULL = identity). A slot outside [0, capacity) is not written and
 * sets err_flag bit 8 (err_flag may be NULL). */
int fg_rope_kv_write(const void* qkv, int dtype, int64_t ld_qkv, int batch, int num_nodes, int q_heads, int kv_heads,
                     int head_dim, const int32_t* seq_len, const int32_t* pos_offset, int64_t pos_batch_stride,
                     const float* inv_freq, void* q_out, void* k_cache, void* v_cache, int64_t cache_batch_stride,
                     int64_t cache_head_stride, int capacity, const int32_t* row_map, int32_t* err_flag,
                     void* stream);

/* Tree attention: node n of sequence b attends to cache keys [0, seq_len[b]) and to
 * tree keys seq_len[b] + m for every bit m of anc[b*anc_batch_stride + n] (num_nodes <= 64).
 * anc == NULL: the new keys form a causal chain, node n sees new keys 0..n (prefill;
 * num_nodes <= 8192). q/out [batch, num_nodes, Hq, d]; bf16 needs d == 128, fp32 d 64 or 128.
 * When batch x kv_heads leaves the chip idle (bf16), each sequence's keys are split over
 * several workgroups whose partial softmax states are merged by a second launch; that
 * needs workspace >= fg_tree_attention_workspace(...) (0 when no split is used; a null
 * or smaller workspace runs unsplit). */
size_t fg_tree_attention_workspace(int batch, int num_nodes, int q_heads, int kv_heads, int head_dim, int capacity);
int fg_tree_attention(const void* q, void* out, const void* k_cache, const void* v_cache, int dtype, int batch,
                      int num_nodes, int q_heads, int kv_heads, int head_dim, int64_t cache_batch_stride,
                      int64_t cache_head_stride, int capacity, const int32_t* seq_len, const int32_t* row_map,
                      const uint64_t* anc, int64_t anc_batch_stride, float scale, void* workspace,
                      size_t workspace_bytes, void* stream);

/* y = RMSNorm(x [+ delta]) * weight over rows of `hidden`; with delta, x += delta first. */
int fg_rmsnorm(void* x, const void* delta, const void* weight, void* y, int dtype, int rows, int hidden, float eps,
               void* stream);
/* out[t, i] = SiLU(gate_up[t, i]) * gate_up[t, inter + i] */
int fg_swiglu(const void* gate_up, void* out, int dtype, int rows, int inter, void* stream);
/* out[t, i] = SiLU(bf16(x[t] . w[i])) * bf16(x[t] . w[inter + i]), i < inter: the gate/up
 * projection (w = [gate; up], [2*inter, hidden] bf16, rows `ldw` apart) with SwiGLU in its
 * epilogue; bf16 x [rows, hidden] (row stride ldx) and out [rows, inter] (row stride ldo).
 * hidden % 64 == 0, inter % 4 == 0; x and w rows 16-byte aligned, out rows 8-byte aligned.
 * tile_rows: 0 (chosen from the shape), 64, 128, 192 or 256 rows per workgroup tile. */
int fg_gate_up_swiglu(const void* x, int64_t ldx, const void* w_gate_up, int64_t ldw, void* out, int64_t ldo, int rows,
                      int inter, int hidden, int tile_rows, void* stream);

/* Split-K projection: part[s][r, c] = sum over split s's k-steps of x[r, k] * w[c, k], fp32
 * (bf16 x [rows, hidden] row stride ldx, w [cols, hidden] row stride ldw; part [splits, rows, cols]
 * contiguous). Replaces the q/k/v, o and down projections (nn.Linear) of the HF decoder layers the
 * reference's tree verify runs: models/qwen_flashgrpo_wrapper.py:172-180. hidden % 64 == 0,
 * cols % 4 == 0, 16-byte aligned rows; splits in [1, hidden/64] with
 * ceil(nk / ceil(nk / splits)) == splits (nk = hidden / 64), so that every split has k-steps;
 * tile_m, tile_n: 64 or 128 output rows / columns per workgroup; stages: 2, 3 or 4 k-steps of
 * 64 in the LDS ring (stages - 1 of them loading while one is computed), 0 for 4. */
int fg_linear_parts(const void* x, int64_t ldx, const void* w, int64_t ldw, float* part, int rows, int cols,
                    int hidden, int splits, int tile_m, int tile_n, int stages, void* stream);

/* The residual add and the following RMSNorm of an O or down projection given as split-K parts
 * [splits, rows, hidden]: x[r] = bf16(x[r] + bf16(sum_s part[s][r])) in place (bf16 x, row stride
 * ldx), then h[r] = weight * bf16(x[r] * rsqrt(mean(x[r]^2) + eps)) (bf16, row stride ldh).
 * Replaces `residual + self_attn(...)` / `residual + mlp(...)` and the next RMSNorm of the HF
 * decoder layer (models/qwen_flashgrpo_wrapper.py:172-180). hidden % 8 == 0, hidden <= 8192. */
int fg_residual_rmsnorm_parts(const float* part, int splits, int rows, int hidden, void* x, int64_t ldx,
                              const void* weight, float eps, void* h, int64_t ldh, void* stream);

/* fg_rope_kv_write with the projected qkv rows given as split-K parts [splits, batch*num_nodes,
 * (q_heads + 2*kv_heads)*head_dim] (fg_linear_parts): each value is bf16(sum_s part + bias) (bias
 * [width] in `dtype`, or NULL), then rotated and written as fg_rope_kv_write does. Replaces the
 * q/k/v projections' bias add with the HF rotary embedding and DynamicCache.update
 * (models/qwen_flashgrpo_wrapper.py:172-180). */
int fg_rope_kv_write_parts(const float* part, int splits, const void* bias, int dtype, int batch, int num_nodes,
                           int q_heads, int kv_heads, int head_dim, const int32_t* seq_len, const int32_t* pos_offset,
                           int64_t pos_batch_stride, const float* inv_freq, void* q_out, void* k_cache, void* v_cache,
                           int64_t cache_batch_stride, int64_t cache_head_stride, int capacity,
                           const int32_t* row_map, int32_t* err_flag, void* stream);

/* table[r][j] = (bf16(cos(a)), bf16(sin(a))) as fp32 pairs, a = (seq_len[b] + pos_offset[b *
 * pos_batch_stride + n]) * inv_freq[j], for rows r = b * num_nodes + n and j < head_dim / 2: the
 * rotary values fg_rope_kv_write computes per token, once per forward for fg_linear_rope_kv_write.
 * Replaces the HF rotary embedding's cos / sin (models/qwen_flashgrpo_wrapper.py:172-180). */
int fg_rope_cos_sin(const int32_t* seq_len, const int32_t* pos_offset, int64_t pos_batch_stride, const float* inv_freq,
                    int batch, int num_nodes, int head_dim, float* table, void* stream);

/* The q/k/v projection of rows = batch*num_nodes bf16 rows x [rows, ldx] (hidden a multiple of 64)
 * with the bias, rotary embedding and KV-slot write in the GEMM's epilogue (one split of
 * fg_linear_parts' kernel, tile_m / tile_n 64 or 128, stages 0 (4), 2, 3 or 4): the same values,
 * bit for bit, as fg_linear_parts with one split followed by fg_rope_kv_write_parts. w_pairs and
 * bias_pairs (NULL for none) are the projection's weight rows and bias with every q and k head's
 * rows pair-interleaved -- row 2j of a head holds its row j, row 2j + 1 its row j + head_dim/2 --
 * and the v heads' rows in order; cos_sin is fg_rope_cos_sin's table of these rows; the outputs
 * are in the usual order. Replaces the q/k/v projections with the HF rotary embedding and
 * DynamicCache.update (models/qwen_flashgrpo_wrapper.py:172-180). */
int fg_linear_rope_kv_write(const void* x, int64_t ldx, const void* w_pairs, int64_t ldw, const void* bias_pairs,
                            int rows, int hidden, int tile_m, int tile_n, int stages, int batch, int num_nodes,
                            int q_heads, int kv_heads, int head_dim, const int32_t* seq_len, const float* cos_sin,
                            void* q_out, void* k_cache, void* v_cache, int64_t cache_batch_stride,
                            int64_t cache_head_stride, int capacity, const int32_t* row_map, int32_t* err_flag,
                            void* stream);

/* out[r] = [LayerNorm(state[r]) * state_w + state_b, LayerNorm(token[r]) * token_w + token_b]
 * ([rows, 2*hidden], row stride 2*hidden): the ChainDraftCell's normalised inputs side by side.
 * Weights and biases in the row dtype; hidden % 8 == 0, hidden <= 8192, 16-byte aligned rows. */
int fg_chain_cell_norm(const void* state, int64_t ld_state, const void* token, int64_t ld_token, int dtype,
                       int rows, int hidden, const void* state_w, const void* state_b, const void* token_w,
                       const void* token_b, float eps, void* out, void* stream);

/* Workspace (bytes) that lets fg_sample_tokens / fg_walk_step split each row of an
 * unrestricted (no top-k, no top-p) or greedy draw over several workgroups. */
size_t fg_sample_workspace(int rows);

/* One supplied-noise draw per row (rule documented in csrc/sample.hip).
 * Row r reads logits row row_index ? row_index[r] : r. forced (optional): a value
 * >= 0 is emitted instead of sampling. Noise: noise[r*noise_stride + noise_col]
 * when noise != NULL, else counter noise (seed, step, seq_ids ? seq_ids[r] : r, draw).
 * greedy or temperature == 0: argmax (first maximum). top_k <= 0: off.
 * top_p_fixed = floor(top_p * 2^32), 0 = off. workspace (optional, >= fg_sample_workspace(rows)
 * bytes): unrestricted and greedy draws then run split over several workgroups per row;
 * results are identical either way. */
int fg_sample_tokens(const void* logits, int dtype, int64_t row_stride, int rows, int vocab,
                     const int32_t* row_index, const int32_t* forced, const uint32_t* noise, int noise_stride,
                     int noise_col, uint64_t seed, uint64_t step, const int32_t* seq_ids, int draw,
                     float temperature, int greedy, int top_k, uint32_t top_p_fixed, int32_t* out_tokens,
                     void* workspace, size_t workspace_bytes, void* stream);

/* fg_sample_tokens without a workspace argument and without any allocation. No
 * counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The split partials live in a static device array of the library (9.1 MB per GPU,
 * held until the process ends) that holds rows <= fg_sample_tokens_noalloc_max_rows()
 * (256); more rows are rejected with an error. Same arguments, rule and tokens as
 * fg_sample_tokens with a large enough workspace. Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (on different streams, or from several
 * threads) race and must be ordered by the caller. */
size_t fg_sample_tokens_noalloc_max_rows(void);
int fg_sample_tokens_noalloc(const void* logits, int dtype, int64_t row_stride, int rows, int vocab,
                             const int32_t* row_index, const int32_t* forced, const uint32_t* noise,
                             int noise_stride, int noise_col, uint64_t seed, uint64_t step, const int32_t* seq_ids,
                             int draw, float temperature, int greedy, int top_k, uint32_t top_p_fixed,
                             int32_t* out_tokens, void* stream);

/* exact_target acceptance walk over `batch` trees (one launch per walk step).
 * Node n of tree b: tree_tokens/parents[b*nmax + n], n < n_nodes[b], root = node 0.
 * Logits of node n: row slot_map[b*nmax + n] of tree_logits (packed internal nodes),
 * or row b*nmax + n when slot_map is NULL (dense). Walk step t (0-based) draws
 * noise[b*noise_stride + noise_col0 + t] or counter noise with draw index draw0 + t.
 * Outputs: acc_tokens/acc_nodes [batch, acc_stride], acc_len, last_node, correction
 * (the unmatched sample, -1 if none). workspace: 3*batch int32 (walk state). err_flag bits:
 * 2 = a walked node had no logits row, 4 = acc_stride too small. */
int fg_accept_walk(const void* tree_logits, int dtype, int64_t row_stride, int vocab, const int32_t* slot_map,
                   const int32_t* tree_tokens, const int32_t* parents, const int32_t* n_nodes, int nmax, int batch,
                   int max_walk_steps, const uint32_t* noise, int noise_stride, int noise_col0, uint64_t seed,
                   uint64_t step, const int32_t* seq_ids, int draw0, float temperature, int greedy, int top_k,
                   uint32_t top_p_fixed, int32_t* acc_tokens, int32_t* acc_nodes, int acc_stride, int32_t* acc_len,
                   int32_t* last_node, int32_t* correction, int32_t* workspace, int32_t* err_flag, void* stream);

/* The same walk one step at a time, for callers that compute each step's logits
 * rows on demand (the LM head of only the nodes the walk actually samples):
 *   fg_walk_begin  -- initialise outputs (acc rows: the root, then zeros) and the walk state (3*batch int32);
 *   fg_walk_rows   -- row_index[b] = b*nmax + current parent of b, row_active[b];
 *   fg_walk_step   -- draw for every active row b from row b of step_logits
 *                     (noise column noise_col0 + walk_step, counter draw draw0 + walk_step).
 * After the walk, state[2*batch + b] is the step whose logits row b last sampled (-1: none).
 * fg_walk_step's workspace is optional, as for fg_sample_tokens (rows = batch). With a
 * workspace, an unrestricted or greedy step whose row maxima parts are given (part_max /
 * part_key [batch, nparts], as fg_lm_head_topk writes them with the step's logits) skips
 * the chunk-maxima launch. next_row_index / next_row_active (optional): the step also writes the next
 * step's rows, as fg_walk_rows would (rows that are already inactive keep their entries). */
int fg_walk_begin(const int32_t* tree_tokens, const int32_t* parents, const int32_t* n_nodes, int nmax, int batch,
                  int32_t* acc_tokens, int32_t* acc_nodes, int acc_stride, int32_t* acc_len, int32_t* last_node,
                  int32_t* correction, int32_t* state, void* stream);
int fg_walk_rows(const int32_t* state, int batch, int nmax, int32_t* row_index, int32_t* row_active, void* stream);
int fg_walk_step(const void* step_logits, int dtype, int64_t row_stride, int vocab, const int32_t* tree_tokens,
                 const int32_t* parents, const int32_t* n_nodes, int nmax, int batch, int walk_step,
                 const uint32_t* noise, int noise_stride, int noise_col0, uint64_t seed, uint64_t step,
                 const int32_t* seq_ids, int draw0, float temperature, int greedy, int top_k, uint32_t top_p_fixed,
                 int32_t* acc_tokens, int32_t* acc_nodes, int acc_stride, int32_t* acc_len, int32_t* last_node,
                 int32_t* correction, int32_t* state, int32_t* err_flag, const float* part_max,
                 const uint64_t* part_key, int nparts, int32_t* next_row_index, int32_t* next_row_active,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Length clamp (max(1, max_length - old_len)), EOS cut (eos_token_id < 0: none),
 * finished flags and, when pending_root != NULL, the next round's forced root
 * (the correction token if the whole raw path was kept and the row continues). */
int fg_accept_finalize(const int32_t* acc_tokens, const int32_t* acc_nodes, int acc_stride, int32_t* acc_len,
                       int32_t* last_node, const int32_t* correction, const int32_t* old_len, int max_length,
                       int eos_token_id, int32_t* finished, int32_t* pending_root, int batch, void* stream);

/* Accepted-path compaction for all layers in one launch: for each of num_tensors
 * cache tensors (device array tensor_ptrs, e.g. K0,V0,K1,V1,...) laid out
 * [Bc, kv_heads, capacity, head_dim] with the given element strides, moves rows
 * seq_len[b] + acc_nodes[b, j] to seq_len[b] + j for j < acc_len[b]. All sources
 * are read before any destination is written. Does not modify seq_len.
 * acc_stride (the longest accepted path) is at most 32.
 * err_flag bit 1: a node index was outside [0, tree_nodes) or a path was longer than the
 * tree (that row is skipped). */
int fg_kv_path_gather(const uint64_t* tensor_ptrs, int num_tensors, int batch, int kv_heads, int head_dim,
                      int elem_bytes, int64_t batch_stride, int64_t head_stride, int64_t row_stride, int capacity,
                      const int32_t* seq_len, const int32_t* row_map, const int32_t* acc_nodes, int acc_stride,
                      const int32_t* acc_len, int tree_nodes, int32_t* err_flag, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHGRPO_AMD_H */
