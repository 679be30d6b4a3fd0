// Per-depth Medusa top-k candidate selection and dense-tree token layout.
//
// Replaces the per-depth torch.topk + .cpu() + Python BFS of
// flashgrpo/decoding/medusa_tree.py:228-278. Candidates are ranked by
// (value desc, index asc) so ties resolve the same way on every run; the
// tree topology (parent, depth, candidate rank of each node) depends only on
// the plan and is supplied by the host, the kernel fills in the tokens.
//
// Phase 1: grid (rows, chunks). Each thread keeps a sorted top-K of 64-bit
// rank keys over its strided elements (and, optionally, a running max and
// sum of exp for the row's log-sum-exp); lists merge across the wave with the
// bitonic "max(A[i], B[K-1-i]) then sort" step, then across waves in LDS.
// Phase 2: one wave per row merges the chunk lists.
//
// With `sanitize` the values are first mapped as torch.nan_to_num(x.float(),
// nan=-1e9, posinf=1e9, neginf=-1e9) does before the chain builder's top-k
// (flashgrpo/decoding/flash_medusa_decoder.py:477-482); without it NaN ranks
// above every number, as in torch.topk.
#include "fg_common.h"
#include "fg_topk.h"

#include <algorithm>
#include <climits>
#include <cmath>

namespace {

using fg::insert_key;
using fg::LseAcc;
using fg::lse_combine;
using fg::merge_desc;
using fg::sanitize;
using fg::wave_merge;

constexpr int kThreads = 256;

template <int DT, int K, bool STATS, bool SAN>
__global__ void __launch_bounds__(kThreads) topk_phase1(const void* __restrict__ logits, int64_t row_stride,
                                                        int vocab, int chunk, uint64_t* __restrict__ part_keys,
                                                        float2* __restrict__ part_lse) {
  const int row = blockIdx.x;
  const int c = blockIdx.y;
  const int nchunks = gridDim.y;
  const char* rowp = (const char*)logits + (int64_t)row * row_stride * (DT == fg::kBF16 ? 2 : 4);
  const int lo = c * chunk;
  const int hi = min(vocab, lo + chunk);
  uint64_t top[K];
#pragma unroll
  for (int i = 0; i < K; ++i) top[i] = 0;
  LseAcc acc{-INFINITY, 0.0f};
  // Vector body: 8 elements per thread per step; chunk starts are multiples of 8.
  const int vec_hi = lo + ((hi - lo) & ~7);
  for (int i = lo + threadIdx.x * 8; i < vec_hi; i += kThreads * 8) {
    float v[8];
    fg::load8<DT>(rowp, i, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = sanitize<SAN>(v[j]);
#pragma unroll
    for (int j = 0; j < 8; ++j) insert_key<K>(top, fg::rank_key(v[j], (uint32_t)(i + j)));
    if constexpr (STATS) {
      float m8 = v[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) m8 = fmaxf(m8, v[j]);
      float m = fmaxf(acc.m, m8);
      float s = (acc.m == -INFINITY) ? 0.0f : acc.s * __expf(acc.m - m);
#pragma unroll
      for (int j = 0; j < 8; ++j) s += __expf(v[j] - m);
      acc = {m, s};
    }
  }
  for (int i = vec_hi + threadIdx.x; i < hi; i += kThreads) {
    float v = sanitize<SAN>(fg::load_elem<DT>(rowp, i));
    insert_key<K>(top, fg::rank_key(v, (uint32_t)i));
    if constexpr (STATS) acc = lse_combine(acc, LseAcc{v, 1.0f});
  }
  wave_merge<K>(top);
  __shared__ uint64_t s_top[kThreads / 64][K];
  __shared__ float2 s_lse[kThreads / 64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if constexpr (STATS) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      LseAcc other{__shfl_xor(acc.m, o, 64), __shfl_xor(acc.s, o, 64)};
      acc = lse_combine(acc, other);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < K; ++i) s_top[wave][i] = top[i];
    s_lse[wave] = make_float2(acc.m, acc.s);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) {
      uint64_t other[K];
#pragma unroll
      for (int i = 0; i < K; ++i) other[i] = s_top[w][i];
      merge_desc<K>(top, other);
      if constexpr (STATS) acc = lse_combine(acc, LseAcc{s_lse[w].x, s_lse[w].y});
    }
    uint64_t* out = part_keys + ((int64_t)row * nchunks + c) * K;
#pragma unroll
    for (int i = 0; i < K; ++i) out[i] = top[i];
    if constexpr (STATS) part_lse[(int64_t)row * nchunks + c] = make_float2(acc.m, acc.s);
  }
}

template <int K, bool STATS>
__global__ void __launch_bounds__(64) topk_phase2(const uint64_t* __restrict__ part_keys,
                                                  const float2* __restrict__ part_lse, int nchunks, int kout,
                                                  int32_t* __restrict__ cand_tokens, float* __restrict__ cand_scores,
                                                  float* __restrict__ row_stats) {
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  uint64_t top[K];
  LseAcc acc{-INFINITY, 0.0f};
#pragma unroll
  for (int i = 0; i < K; ++i) top[i] = 0;
  for (int c = lane; c < nchunks; c += 64) {
    uint64_t other[K];
    const uint64_t* in = part_keys + ((int64_t)row * nchunks + c) * K;
#pragma unroll
    for (int i = 0; i < K; ++i) other[i] = in[i];
    merge_desc<K>(top, other);
    if constexpr (STATS) {
      float2 p = part_lse[(int64_t)row * nchunks + c];
      acc = lse_combine(acc, LseAcc{p.x, p.y});
    }
  }
  wave_merge<K>(top);
  if constexpr (STATS) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      LseAcc other{__shfl_xor(acc.m, o, 64), __shfl_xor(acc.s, o, 64)};
      acc = lse_combine(acc, other);
    }
  }
  if (lane == 0) {
    for (int i = 0; i < kout; ++i) {
      cand_tokens[(int64_t)row * kout + i] = (int32_t)fg::rank_key_index(top[i]);
      cand_scores[(int64_t)row * kout + i] = fg::rank_key_value(top[i]);
    }
    if constexpr (STATS) {
      row_stats[2 * row] = acc.m;
      row_stats[2 * row + 1] = acc.m + __logf(acc.s);
    }
  }
}

template <int DT, int K, bool STATS>
void launch_topk(const void* logits, int64_t row_stride, int rows, int vocab, int chunks, int chunk, int kout,
                 uint64_t* part_keys, float2* part_lse, int32_t* tok, float* score, float* stats, bool san,
                 hipStream_t stream) {
  if (san)
    hipLaunchKernelGGL((topk_phase1<DT, K, STATS, true>), dim3(rows, chunks), dim3(kThreads), 0, stream, logits,
                       row_stride, vocab, chunk, part_keys, part_lse);
  else
    hipLaunchKernelGGL((topk_phase1<DT, K, STATS, false>), dim3(rows, chunks), dim3(kThreads), 0, stream, logits, row_stride,
                     vocab, chunk, part_keys, part_lse);
  hipLaunchKernelGGL((topk_phase2<K, STATS>), dim3(rows), dim3(64), 0, stream, part_keys, part_lse, chunks, kout, tok,
                     score, stats);
}

template <int DT, bool STATS>
void dispatch_k(int K, const void* logits, int64_t row_stride, int rows, int vocab, int chunks, int chunk, int kout,
                uint64_t* pk, float2* pl, int32_t* tok, float* score, float* stats, bool san, hipStream_t s) {
  switch (K) {
    case 1: launch_topk<DT, 1, STATS>(logits, row_stride, rows, vocab, chunks, chunk, kout, pk, pl, tok, score, stats, san, s); break;
    case 2: launch_topk<DT, 2, STATS>(logits, row_stride, rows, vocab, chunks, chunk, kout, pk, pl, tok, score, stats, san, s); break;
    case 4: launch_topk<DT, 4, STATS>(logits, row_stride, rows, vocab, chunks, chunk, kout, pk, pl, tok, score, stats, san, s); break;
    case 8: launch_topk<DT, 8, STATS>(logits, row_stride, rows, vocab, chunks, chunk, kout, pk, pl, tok, score, stats, san, s); break;
    default: launch_topk<DT, 16, STATS>(logits, row_stride, rows, vocab, chunks, chunk, kout, pk, pl, tok, score, stats, san, s); break;
  }
}

__global__ void tree_layout_kernel(const int32_t* __restrict__ cand_tokens, const float* __restrict__ cand_scores,
                                   int kstride, int batch, const int32_t* __restrict__ roots,
                                   const int32_t* __restrict__ node_depth, const int32_t* __restrict__ node_rank,
                                   int num_nodes, int32_t* __restrict__ tree_tokens, float* __restrict__ tree_scores,
                                   int out_stride) {
  const int b = blockIdx.x;
  for (int n = threadIdx.x; n < num_nodes; n += blockDim.x) {
    int32_t tok;
    float sc;
    if (n == 0) {
      tok = roots[b];
      sc = 0.0f;
    } else {
      int64_t r = (int64_t)(node_depth[n] - 2) * batch + b;
      tok = cand_tokens[r * kstride + node_rank[n]];
      sc = cand_scores[r * kstride + node_rank[n]];
    }
    tree_tokens[(int64_t)b * out_stride + n] = tok;
    if (tree_scores) tree_scores[(int64_t)b * out_stride + n] = sc;
  }
}

// ---------------------------------------------------------------- sparse asymmetric trees
// One wave per sequence assembles the tree of
// flashgrpo_b200/decoding/medusa_tree.py:549-685 from the per-head top-k lists:
// head-1 nodes under the root, then head-2 and head-3 nodes picked greedily from
// (parent, candidate) pairs (:509-546), then leftover head-1 candidates. A pick is
// the pair of largest parent score + candidate score - penalty * (picks of its
// parent) in float64, the lowest pair index on ties (the reference's first strict
// maximum in parent-major order); a value that is NaN or -inf is never picked. The
// lanes hold the pairs (index lane + 64c) and reduce the best one across the wave.
constexpr int kSpMaxNodes = 128;  // nodes assembled before the budget cut
constexpr int kSpMaxParents = 64;
constexpr int kSpMaxPool = 1024;  // (parent, candidate) pairs of one head
// parents of one head x candidates per parent (kstride <= 16, host-checked): 16 pairs per lane
static_assert(kSpMaxPool == kSpMaxParents * 16 && kSpMaxPool == 64 * 16, "sparse pick pool");

struct SparseArgs {
  const int32_t* cand_tokens;
  const float* cand_scores;
  int kstride, batch;
  const int32_t* roots;
  const uint8_t* gate;
  int n1, n2, n3, realloc, w1, w2, w3, heads, budget, num_nodes;
  float temperature;
  double penalty;
  int32_t *tokens, *parents, *depth, *pos_offset, *n_children, *n_nodes;
  uint64_t* anc;
  double* scores;
};

#pragma clang fp contract(off)
__global__ void __launch_bounds__(64) sparse_tree_kernel(SparseArgs a) {
  __shared__ int tok[kSpMaxNodes], par[kSpMaxNodes], dep[kSpMaxNodes];
  __shared__ double sc[kSpMaxNodes];
  __shared__ int uses[kSpMaxParents];
  const int b = blockIdx.x, lane = threadIdx.x;
  auto row = [&](int h) { return ((int64_t)h * a.batch + b) * a.kstride; };
  auto cand_score = [&](int h, int c) -> double { return (double)(a.cand_scores[row(h) + c] / a.temperature); };
  int cnt = 1;
  if (lane == 0) {
    tok[0] = a.roots[b];
    par[0] = -1;
    dep[0] = 1;
    sc[0] = 0.0;
  }
  const int n1 = min(a.n1, a.w1);
  if (lane < n1) {
    tok[1 + lane] = a.cand_tokens[row(0) + lane];
    par[1 + lane] = 0;
    dep[1 + lane] = 2;
    sc[1 + lane] = cand_score(0, lane);
  }
  cnt += n1;
  __syncthreads();

  // Greedy picks of `count` pairs from parents [p0, p0 + np) x candidates [0, w) of head h.
  auto pick = [&](int h, int p0, int np, int w, int count, int depth) {
    const int P = np * w;
    uint32_t picked = 0;
    if (lane < np) uses[lane] = 0;
    __syncthreads();
    const int npick = min(count, P);
    for (int it = 0; it < npick; ++it) {
      double bv = -INFINITY;
      int bi = INT_MAX;
      for (int c = 0; c * 64 < P; ++c) {
        const int i = lane + 64 * c;
        if (i < P && !((picked >> c) & 1u)) {
          const int j = i / w, r = i - j * w;
          const double cum = sc[p0 + j] + cand_score(h, r);
          const double v = cum - a.penalty * (double)uses[j];
          if (v > bv) {
            bv = v;
            bi = i;
          }
        }
      }
      for (int off = 32; off >= 1; off >>= 1) {
        const double ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (bi == INT_MAX) break;  // wave-uniform: nothing left above -inf
      if (lane == (bi & 63)) picked |= 1u << (bi >> 6);
      const int j = bi / w, r = bi - j * w;
      if (lane == 0) {
        if (cnt < kSpMaxNodes) {
          tok[cnt] = a.cand_tokens[row(h) + r];
          par[cnt] = p0 + j;
          dep[cnt] = depth;
          sc[cnt] = sc[p0 + j] + cand_score(h, r);
        }
        uses[j] += 1;
      }
      ++cnt;
      __syncthreads();
    }
  };

  const bool use3 = a.heads >= 3 && a.n3 > 0 && (!a.gate || a.gate[b]);
  const int n2 = a.n2 + (use3 ? 0 : a.realloc);
  const int h2_begin = cnt;
  if (a.heads >= 2 && n2 > 0) pick(1, 1, n1, a.w2, n2, 3);
  const int h2_end = min(cnt, kSpMaxNodes);
  if (use3 && h2_end > h2_begin) pick(2, h2_begin, h2_end - h2_begin, a.w3, a.n3, 4);
  // leftover head-1 candidates while the budget allows (distinct from every head-1 node)
  if (lane == 0) {
    const int extra_begin = cnt;
    for (int c = n1; c < a.w1 && cnt < a.budget && cnt < kSpMaxNodes; ++c) {
      const int t = a.cand_tokens[row(0) + c];
      bool seen = false;
      for (int m = 1; m <= n1; ++m) seen |= tok[m] == t;
      for (int m = extra_begin; m < cnt; ++m) seen |= tok[m] == t;
      if (seen) continue;
      tok[cnt] = t;
      par[cnt] = 0;
      dep[cnt] = 2;
      sc[cnt] = cand_score(0, c);
      ++cnt;
    }
  }
  __syncthreads();
  cnt = __shfl(cnt, 0);
  const int count = min(min(cnt, a.budget), a.num_nodes);
  const int64_t o = (int64_t)b * a.num_nodes;
  for (int n = lane; n < a.num_nodes; n += 64) {
    if (n < count) {
      uint64_t m = 1ull << n;
      for (int p = par[n]; p >= 0; p = par[p]) m |= 1ull << p;
      int kids = 0;
      for (int c = n + 1; c < count; ++c) kids += par[c] == n;
      a.tokens[o + n] = tok[n];
      a.parents[o + n] = par[n];
      a.depth[o + n] = dep[n];
      a.pos_offset[o + n] = dep[n] - 1;
      a.anc[o + n] = m;
      a.n_children[o + n] = kids;
      if (a.scores) a.scores[o + n] = sc[n];
    } else {
      a.tokens[o + n] = 0;
      a.parents[o + n] = -1;
      a.depth[o + n] = 0;
      a.pos_offset[o + n] = 0;
      a.anc[o + n] = 1ull << n;
      a.n_children[o + n] = 0;
      if (a.scores) a.scores[o + n] = 0.0;
    }
  }
  if (lane == 0) a.n_nodes[b] = count;
}
#pragma clang fp contract(on)

}  // namespace

namespace fg {
int topk_merge_parts(int K, const uint64_t* part_keys, const float2* part_lse, int rows, int nparts, int kout,
                     int32_t* cand_tokens, float* cand_scores, float* row_stats, hipStream_t s) {
  const bool stats = row_stats != nullptr;
#define FG_MERGE(KK)                                                                                          \
  if (stats)                                                                                                  \
    hipLaunchKernelGGL((topk_phase2<KK, true>), dim3(rows), dim3(64), 0, s, part_keys, part_lse, nparts, kout,  \
                       cand_tokens, cand_scores, row_stats);                                                  \
  else                                                                                                        \
    hipLaunchKernelGGL((topk_phase2<KK, false>), dim3(rows), dim3(64), 0, s, part_keys, part_lse, nparts, kout, \
                       cand_tokens, cand_scores, row_stats);
  switch (K) {
    case 1: FG_MERGE(1) break;
    case 2: FG_MERGE(2) break;
    case 4: FG_MERGE(4) break;
    case 8: FG_MERGE(8) break;
    case 16: FG_MERGE(16) break;
    default: return fail("topk_merge_parts: K must be 1, 2, 4, 8 or 16");
  }
#undef FG_MERGE
  return check_launch("topk merge");
}
}  // namespace fg

extern "C" {

// Workspace bytes fg_medusa_topk needs for `rows` rows.
size_t fg_medusa_topk_workspace(int rows, int vocab, int kmax) {
  int chunks = 64;
  return (size_t)rows * chunks * (16 * sizeof(uint64_t) + sizeof(float2)) + 256;
}

int fg_medusa_topk(const void* logits, int dtype, int64_t row_stride, int rows, int vocab, int kmax, int sanitize,
                   int32_t* cand_tokens, float* cand_scores, float* row_stats, void* workspace,
                   size_t workspace_bytes, void* stream) {
  FG_REQUIRE(logits && cand_tokens && cand_scores && workspace, "fg_medusa_topk: null pointer");
  FG_REQUIRE(rows > 0 && vocab > 0 && vocab < (1 << 30), "fg_medusa_topk: bad shape");
  FG_REQUIRE(kmax >= 1 && kmax <= 16 && kmax <= vocab, "fg_medusa_topk: kmax must be in [1, min(16, vocab)]");
  FG_REQUIRE(dtype == fg::kF32 || dtype == fg::kBF16, "fg_medusa_topk: dtype");
  FG_REQUIRE(row_stride >= vocab && row_stride % 8 == 0, "fg_medusa_topk: row_stride must be >= vocab and a multiple of 8");
  FG_REQUIRE(((uintptr_t)logits & 31) == 0, "fg_medusa_topk: logits must be 32-byte aligned");
  int K = kmax <= 1 ? 1 : kmax <= 2 ? 2 : kmax <= 4 ? 4 : kmax <= 8 ? 8 : 16;
  // Enough workgroups to cover the chip: ~2048 in total, chunks of >= 2048 elements.
  int chunks = (2048 + rows - 1) / rows;
  chunks = std::max(1, std::min(chunks, std::min(64, (vocab + 2047) / 2048)));
  int chunk = ((vocab + chunks - 1) / chunks + 7) & ~7;
  chunks = (vocab + chunk - 1) / chunk;
  size_t need = (size_t)rows * chunks * (K * sizeof(uint64_t) + sizeof(float2));
  FG_REQUIRE(workspace_bytes >= need, "fg_medusa_topk: workspace too small");
  uint64_t* pk = (uint64_t*)workspace;
  float2* pl = (float2*)(pk + (size_t)rows * chunks * K);
  hipStream_t s = (hipStream_t)stream;
  bool stats = row_stats != nullptr;
  if (dtype == fg::kBF16) {
    if (stats) dispatch_k<fg::kBF16, true>(K, logits, row_stride, rows, vocab, chunks, chunk, kmax, pk, pl, cand_tokens, cand_scores, row_stats, sanitize != 0, s);
    else dispatch_k<fg::kBF16, false>(K, logits, row_stride, rows, vocab, chunks, chunk, kmax, pk, pl, cand_tokens, cand_scores, row_stats, sanitize != 0, s);
  } else {
    if (stats) dispatch_k<fg::kF32, true>(K, logits, row_stride, rows, vocab, chunks, chunk, kmax, pk, pl, cand_tokens, cand_scores, row_stats, sanitize != 0, s);
    else dispatch_k<fg::kF32, false>(K, logits, row_stride, rows, vocab, chunks, chunk, kmax, pk, pl, cand_tokens, cand_scores, row_stats, sanitize != 0, s);
  }
  return fg::check_launch("fg_medusa_topk");
}

int fg_tree_layout(const int32_t* cand_tokens, const float* cand_scores, int kstride, int batch,
                   const int32_t* roots, const int32_t* node_depth, const int32_t* node_rank, int num_nodes,
                   int32_t* tree_tokens, float* tree_scores, int out_stride, void* stream) {
  FG_REQUIRE(roots && node_depth && node_rank && tree_tokens, "fg_tree_layout: null pointer");
  FG_REQUIRE(batch > 0 && num_nodes > 0 && out_stride >= num_nodes, "fg_tree_layout: bad shape");
  FG_REQUIRE(num_nodes == 1 || (cand_tokens && cand_scores && kstride > 0), "fg_tree_layout: candidates missing");
  hipLaunchKernelGGL(tree_layout_kernel, dim3(batch), dim3(64), 0, (hipStream_t)stream, cand_tokens, cand_scores,
                     kstride, batch, roots, node_depth, node_rank, num_nodes, tree_tokens, tree_scores, out_stride);
  return fg::check_launch("fg_tree_layout");
}

int fg_sparse_tree_layout(const int32_t* cand_tokens, const float* cand_scores, int kstride, int batch,
                          int vocab, const int32_t* roots, const uint8_t* head3_gate, const int32_t* nodes_by_head,
                          int heads, int budget, float temperature, double diversity_penalty, int num_nodes,
                          int32_t* tree_tokens, int32_t* parents, int32_t* depth, int32_t* pos_offset,
                          uint64_t* anc, int32_t* n_children, int32_t* n_nodes, double* scores, void* stream) {
  FG_REQUIRE(cand_tokens && cand_scores && roots && nodes_by_head && tree_tokens && parents && depth && pos_offset &&
                 anc && n_children && n_nodes,
             "fg_sparse_tree_layout: null pointer");
  FG_REQUIRE(batch > 0 && heads >= 1 && vocab >= 1 && kstride >= 1 && kstride <= 16, "fg_sparse_tree_layout: bad shape");
  FG_REQUIRE(num_nodes >= 1 && num_nodes <= 64 && budget >= 1, "fg_sparse_tree_layout: num_nodes must be in [1, 64]");
  FG_REQUIRE(temperature > 0.0f && diversity_penalty >= 0.0, "fg_sparse_tree_layout: temperature must be > 0, penalty >= 0");
  SparseArgs a{};
  a.n1 = nodes_by_head[0];
  a.n2 = heads >= 2 ? nodes_by_head[1] : 0;
  a.n3 = heads >= 3 ? nodes_by_head[2] : 0;
  FG_REQUIRE(a.n1 >= 0 && a.n2 >= 0 && a.n3 >= 0, "fg_sparse_tree_layout: negative node count");
  a.realloc = heads >= 3 ? a.n3 : 0;
  // candidates per head (flashgrpo_b200/decoding/medusa_tree.py:569-579)
  a.w1 = std::max(1, std::min(a.n1 + a.realloc, vocab));
  a.w2 = std::max(1, std::min(a.n2 + a.realloc, vocab));
  a.w3 = std::max(1, std::min(a.n3, vocab));
  FG_REQUIRE(a.w1 <= kstride && (heads < 2 || a.w2 <= kstride) && (heads < 3 || a.w3 <= kstride),
             "fg_sparse_tree_layout: candidate lists (kstride) shorter than the head widths");
  FG_REQUIRE(a.n2 + a.realloc <= kSpMaxParents && 1 + a.n1 + a.n2 + a.n3 + 2 * a.realloc <= kSpMaxNodes,
             "fg_sparse_tree_layout: node counts too large");
  a.cand_tokens = cand_tokens;
  a.cand_scores = cand_scores;
  a.kstride = kstride;
  a.batch = batch;
  a.roots = roots;
  a.gate = head3_gate;
  a.heads = std::min(heads, 3);
  a.budget = budget;
  a.num_nodes = num_nodes;
  a.temperature = temperature;
  a.penalty = diversity_penalty;
  a.tokens = tree_tokens;
  a.parents = parents;
  a.depth = depth;
  a.pos_offset = pos_offset;
  a.anc = anc;
  a.n_children = n_children;
  a.n_nodes = n_nodes;
  a.scores = scores;
  hipLaunchKernelGGL(sparse_tree_kernel, dim3(batch), dim3(64), 0, (hipStream_t)stream, a);
  return fg::check_launch("fg_sparse_tree_layout");
}

}  // extern "C"
