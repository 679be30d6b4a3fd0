// Supplied-noise target sampling and the exact_target acceptance walk.
//
// Replaces sample_from_logits / exact_accept_paths_batch
// (flashgrpo/decoding/acceptance.py:34-130, 179-260; correction tokens as in
// flashgrpo_b200/decoding/acceptance.py:184-267). torch.multinomial cannot take
// caller noise, so the draw follows one integer inverse-CDF rule that the CPU
// oracle reproduces bit for bit:
//   m = max x (NaN ignored), q_i = weight_q40(m, x_i, kt): 2^40 * 2^-(a_i / 2^20) for the
//   fixed-point exponent a_i = trunc((m - x_i) * fp32(2^20 / ln 2) / T) (fg_common.h)
//   candidate order (key(x) desc, index asc); top_k keeps the first k; top_p
//   keeps position j while the preceding kept mass <= floor(total * tp32 / 2^32)
//   target = floor(total_kept * u32 / 2^32); token = first kept index (vocab
//   order) whose inclusive q prefix exceeds target.
// Integer sums make every result independent of reduction order.
//
// Unrestricted and greedy draws with a workspace run split over 16 chunks per
// row (chunk maxima, then one draw launch; a walk step whose row maxima come from
// the LM head's epilogue is the draw launch alone, see "split sampling"), top-p
// draws without top-k over seven launches (see "split top-p"). Otherwise: one
// 1024-thread workgroup per sampled row. The row is split into 16
// contiguous wave segments; a wave walks its segment 512 elements (8 per lane,
// 16-byte loads) per step. Top-k / top-p use an MSB-first 4 x 8-bit radix
// select over the keys with count or q-weighted histograms in LDS.
#include <mutex>

#include "fg_common.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kStep = 512;  // elements per wave step

struct Shared {
  uint64_t exp2[1024];  // kExp2Table
  uint64_t wsum[kWaves];
  uint64_t hist[256];
  uint64_t wkey[kWaves];
  float wmax[kWaves];
  uint64_t u64b[2];
  int32_t i32b[2];
};

template <int DT>
struct Row {
  const char* p;
  int V;
  int seg;
  float kt;             // weight scale: fp32(2^20 / ln 2) / T
  const uint64_t* tbl;  // kExp2Table in LDS
  float m;              // row maximum (NaN ignored)

  FG_DEVICE int load(int i0, float (&x)[8]) const {
    if (i0 + 8 <= V) {
      fg::load8<DT>(p, i0, x);
      return 8;
    }
    int n = V - i0;
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = j < n ? fg::load_elem<DT>(p, i0 + j) : 0.0f;
    return n < 0 ? 0 : n;
  }
  // candidates are ranked by the logits themselves (the temperature scales the weight)
  FG_DEVICE float scaled(float x) const { return x; }
  FG_DEVICE uint64_t weight(float s) const { return fg::weight_q40(m, s, kt, tbl); }
};

// Candidate-set predicate: key > kappa, or key == kappa and index <= last.
struct KeyCut {
  uint32_t kappa;
  uint32_t last;
  FG_DEVICE bool operator()(uint32_t key, uint32_t i) const { return key > kappa || (key == kappa && i <= last); }
};
constexpr KeyCut kAll{0u, 0xffffffffu};

// Calls f(i, s, key) for each element of this wave's segment, 8 per lane per step.
template <int DT, class F>
FG_DEVICE void for_wave_segment(const Row<DT>& r, F&& f) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lo = wave * r.seg;
  const int hi = min(r.V, lo + r.seg);
  for (int base = lo; base < hi; base += kStep) {
    int i0 = base + lane * 8;
    float x[8];
    int n = r.load(i0, x);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < n) {
        float s = r.scaled(x[j]);
        f(i0 + j, s, fg::sort_key32(s));
      }
  }
}

// Elements equal to kappa inside a candidate cut.
struct TiePred {
  KeyCut within;
  uint32_t kappa;
  FG_DEVICE bool operator()(uint32_t key, uint32_t i) const { return key == kappa && within(key, i); }
};

// Block sum over pred-elements of w (1 or q); per-wave partials land in sh.wsum.
template <bool WEIGHTED, int DT, class Pred>
FG_DEVICE uint64_t block_sum(const Row<DT>& r, Pred pred, Shared& sh) {
  __syncthreads();
  uint64_t acc = 0;
  for_wave_segment(r, [&](int i, float s, uint32_t key) {
    if (pred(key, (uint32_t)i)) acc += WEIGHTED ? r.weight(s) : 1ull;
  });
  acc = fg::wave_sum_u64(acc);
  if ((threadIdx.x & 63) == 0) sh.wsum[threadIdx.x >> 6] = acc;
  __syncthreads();
  uint64_t tot = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) tot += sh.wsum[w];
  return tot;
}

// First index (vocabulary order) among pred-elements whose inclusive running
// sum of w exceeds target (-1 if none). sh.wsum must hold the per-wave sums of
// the same (pred, w), as left by block_sum.
template <bool WEIGHTED, int DT, class Pred>
FG_DEVICE int block_locate(const Row<DT>& r, Pred pred, uint64_t target, Shared& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint64_t before = 0;
  int win = -1;
  for (int w = 0; w < kWaves; ++w) {
    if (before + sh.wsum[w] > target) {
      win = w;
      break;
    }
    before += sh.wsum[w];
  }
  __syncthreads();
  if (threadIdx.x == 0) sh.i32b[0] = -1;
  __syncthreads();
  if (wave == win) {
    uint64_t run = before;
    const int lo = wave * r.seg;
    const int hi = min(r.V, lo + r.seg);
    for (int base = lo; base < hi; base += kStep) {
      int i0 = base + lane * 8;
      float x[8];
      int n = r.load(i0, x);
      uint64_t w8[8];
      uint64_t mine = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        w8[j] = 0;
        if (j < n) {
          float s = r.scaled(x[j]);
          if (pred(fg::sort_key32(s), (uint32_t)(i0 + j))) w8[j] = WEIGHTED ? r.weight(s) : 1ull;
        }
        mine += w8[j];
      }
      uint64_t incl = fg::wave_incl_scan_u64(mine);
      uint64_t step_total = fg::shfl_u64(incl, 63);
      if (run + step_total > target) {
        uint64_t excl = run + incl - mine;
        if (excl <= target && target < run + incl) {
          uint64_t c = excl;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            c += w8[j];
            if (c > target) {
              sh.i32b[0] = i0 + j;
              break;
            }
          }
        }
        break;
      }
      run += step_total;
    }
  }
  __syncthreads();
  return sh.i32b[0];
}

// MSB-first radix select over `within`-elements in candidate order
// (key desc, index asc): returns the cut that keeps every position up to and
// including the first one where the running count / q-mass exceeds target.
template <bool WEIGHTED, int DT>
FG_DEVICE KeyCut radix_select(const Row<DT>& r, KeyCut within, uint64_t target, Shared& sh) {
  uint32_t prefix = 0, pmask = 0;
  uint64_t above = 0;  // mass of within-elements whose key is above the current range
  const int lane = threadIdx.x & 63;
  for (int level = 0; level < 4; ++level) {
    const int shift = 24 - 8 * level;
    __syncthreads();
    for (int d = threadIdx.x; d < 256; d += kThreads) sh.hist[d] = 0;
    __syncthreads();
    for_wave_segment(r, [&](int i, float s, uint32_t key) {
      if (within(key, (uint32_t)i) && (key & pmask) == prefix)
        atomicAdd((unsigned long long*)&sh.hist[(key >> shift) & 255u],
                  (unsigned long long)(WEIGHTED ? r.weight(s) : 1ull));
    });
    __syncthreads();
    if (threadIdx.x < 64) {
      // lane l owns digits 255-4l .. 252-4l, scanned from the largest digit down
      uint64_t h[4], mine = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        h[j] = sh.hist[255 - 4 * lane - j];
        mine += h[j];
      }
      uint64_t incl = fg::wave_incl_scan_u64(mine);
      uint64_t excl = incl - mine;
      if (above + excl <= target && target < above + incl) {
        uint64_t c = above + excl;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (c + h[j] > target) {
            sh.i32b[1] = 255 - 4 * lane - j;
            sh.u64b[1] = c;
            break;
          }
          c += h[j];
        }
      }
    }
    __syncthreads();
    prefix |= (uint32_t)sh.i32b[1] << shift;
    above = sh.u64b[1];
    pmask |= 255u << shift;
  }
  // Ties on the selected key resolve in index order.
  TiePred tie{within, prefix};
  block_sum<WEIGHTED, DT>(r, tie, sh);
  int last = block_locate<WEIGHTED, DT>(r, tie, target - above, sh);
  return KeyCut{prefix, (uint32_t)last};
}

// First maximum of the raw logits (rank keys: value desc, index asc).
template <int DT>
FG_DEVICE int block_argmax(const Row<DT>& raw, Shared& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint64_t best = 0;
  for_wave_segment(raw, [&](int i, float, uint32_t key) {
    uint64_t k = ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
    best = k > best ? k : best;
  });
  best = fg::wave_max_u64(best);
  __syncthreads();
  if (lane == 0) sh.wkey[wave] = best;
  __syncthreads();
  uint64_t b = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) b = sh.wkey[w] > b ? sh.wkey[w] : b;
  return (int)fg::rank_key_index(b);
}

struct SampleParams {
  float temperature;
  int greedy;
  int top_k;      // 0 = off
  uint32_t tp32;  // 0 = off
};

// One draw from one row by the whole block. Returns the token (all threads).
template <int DT>
FG_DEVICE int block_sample(const void* rowp, int V, const SampleParams& sp, uint32_t u, Shared& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  Row<DT> r;
  r.p = (const char*)rowp;
  r.V = V;
  r.seg = (((V + kWaves - 1) / kWaves) + kStep - 1) / kStep * kStep;
  r.kt = fg::weight_kt(sp.temperature > 0.0f && sp.temperature != 1.0f, sp.temperature);
  r.tbl = sh.exp2;
  r.m = 0.0f;
  if (sp.greedy) return block_argmax<DT>(r, sh);
  fg::exp2_table_to_lds(sh.exp2);  // visible after the barriers of the max below
  float mx = -INFINITY;
  for_wave_segment(r, [&](int, float s, uint32_t) { mx = fmaxf(mx, s); });
  mx = fg::wave_max(mx);
  __syncthreads();
  if (lane == 0) sh.wmax[wave] = mx;
  __syncthreads();
  mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, sh.wmax[w]);
  r.m = mx;

  KeyCut keep = kAll;
  if (sp.top_k > 0) keep = radix_select<false, DT>(r, kAll, (uint64_t)(sp.top_k - 1), sh);
  if (sp.tp32) {
    uint64_t tot = block_sum<true, DT>(r, keep, sh);
    keep = radix_select<true, DT>(r, keep, fg::mulhi_u64_u32(tot, sp.tp32), sh);
  }
  uint64_t total = block_sum<true, DT>(r, keep, sh);
  if (total == 0) return block_argmax<DT>(r, sh);
  return block_locate<true, DT>(r, keep, fg::mulhi_u64_u32(total, u), sh);
}

FG_DEVICE uint32_t noise_value(const uint32_t* noise, int64_t noise_index, uint64_t seed, uint64_t step,
                               uint32_t seq, uint32_t draw) {
  if (noise) return noise[noise_index];
  return fg::counter_noise(seed, step, seq, draw);
}

template <int DT>
__global__ void __launch_bounds__(kThreads) sample_rows_kernel(
    const void* __restrict__ logits, int64_t row_stride, int vocab, const int32_t* __restrict__ row_index,
    const int32_t* __restrict__ forced, const uint32_t* __restrict__ noise, int noise_stride, int noise_col,
    uint64_t seed, uint64_t step, const int32_t* __restrict__ seq_ids, int draw, SampleParams sp,
    int32_t* __restrict__ out) {
  __shared__ Shared sh;
  const int rrow = blockIdx.x;
  if (forced && forced[rrow] >= 0) {
    if (threadIdx.x == 0) out[rrow] = forced[rrow];
    return;
  }
  const int src = row_index ? row_index[rrow] : rrow;
  const char* rowp = (const char*)logits + (int64_t)src * row_stride * (DT == fg::kBF16 ? 2 : 4);
  uint32_t seq = seq_ids ? (uint32_t)seq_ids[rrow] : (uint32_t)rrow;
  uint32_t u = noise_value(noise, (int64_t)rrow * noise_stride + noise_col, seed, step, seq, (uint32_t)draw);
  int tok = block_sample<DT>(rowp, vocab, sp, u, sh);
  if (threadIdx.x == 0) out[rrow] = tok;
}

// Walk state lives in the caller's workspace: parent[B], active[B], and the
// walk step at which each row last sampled (-1 before its first draw) [B].
__global__ void walk_init_kernel(const int32_t* __restrict__ tree_tokens, const int32_t* __restrict__ parents,
                                 const int32_t* __restrict__ n_nodes, int nmax, int batch, int32_t* acc_tokens,
                                 int32_t* acc_nodes, int acc_stride, int32_t* acc_len, int32_t* last_node,
                                 int32_t* correction, int32_t* state) {
  int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  acc_tokens[(int64_t)b * acc_stride] = tree_tokens[(int64_t)b * nmax];
  acc_nodes[(int64_t)b * acc_stride] = 0;
  for (int j = 1; j < acc_stride; ++j) {  // the rest of the rows start at 0
    acc_tokens[(int64_t)b * acc_stride + j] = 0;
    acc_nodes[(int64_t)b * acc_stride + j] = 0;
  }
  acc_len[b] = 1;
  last_node[b] = 0;
  correction[b] = -1;
  int has_child = 0;
  for (int c = 1; c < n_nodes[b]; ++c) has_child |= parents[(int64_t)b * nmax + c] == 0;
  state[b] = 0;                  // parent
  state[batch + b] = has_child;  // active
  state[2 * batch + b] = -1;     // last sampling step
}

// Lazy LM-head rows of a walk step: row b samples from hidden row b*nmax + parent[b].
__global__ void walk_rows_kernel(const int32_t* __restrict__ state, int batch, int nmax, int32_t* row_index,
                                 int32_t* row_active) {
  int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  row_index[b] = b * nmax + state[b];
  row_active[b] = state[batch + b];
}

// Walk update of tree b after its draw `tok` at `parent`, by the 64 lanes of one wave
// (nmax <= 64, host-checked): lane c loads node c's parent and token, one ballot finds the
// first child of `parent` drawing `tok` (the lowest such node index) and a second whether
// that child has children; lane 0 writes the results. A serial scan by one thread would
// wait for up to 2 nmax dependent loads. tok and parent are taken from lane 0.
// next_rows / next_active (optional): the LM-head rows of the next walk step of tree b,
// as walk_rows_kernel would write them.
FG_DEVICE void walk_apply(int b, int tok, int parent, const int32_t* tree_tokens, const int32_t* parents,
                          const int32_t* n_nodes, int nmax, int batch, int walk_step, int32_t* acc_tokens,
                          int32_t* acc_nodes, int acc_stride, int32_t* acc_len, int32_t* last_node,
                          int32_t* correction, int32_t* state, int32_t* err_flag, int32_t* next_rows = nullptr,
                          int32_t* next_active = nullptr) {
  const int lane = threadIdx.x & 63;
  tok = __builtin_amdgcn_readfirstlane(tok);
  parent = __builtin_amdgcn_readfirstlane(parent);
  const int nn = n_nodes[b];
  const bool in = lane >= 1 && lane < nn;
  const int pc = in ? parents[(int64_t)b * nmax + lane] : -2;
  const int tc = in ? tree_tokens[(int64_t)b * nmax + lane] : 0;
  const uint64_t hit = __ballot(in && pc == parent && tc == tok);
  const int match = hit ? (int)__builtin_ctzll(hit) : -1;
  const uint64_t kids = __ballot(in && match >= 0 && lane > match && pc == match);
  if (lane != 0) return;
  state[2 * batch + b] = walk_step;
  if (match < 0) {
    correction[b] = tok;
    state[batch + b] = 0;
  } else {
    int len = acc_len[b];
    if (len < acc_stride) {
      acc_tokens[(int64_t)b * acc_stride + len] = tok;
      acc_nodes[(int64_t)b * acc_stride + len] = match;
      acc_len[b] = len + 1;
    } else if (err_flag) {
      atomicOr(err_flag, 4);
    }
    last_node[b] = match;
    state[b] = match;
    state[batch + b] = kids != 0ull;
  }
  if (next_rows) {
    next_rows[b] = b * nmax + state[b];
    next_active[b] = state[batch + b];
  }
}

template <int DT>
__global__ void __launch_bounds__(kThreads) walk_step_kernel(
    const void* __restrict__ logits, int64_t row_stride, int vocab, const int32_t* __restrict__ slot_map,
    const int32_t* __restrict__ tree_tokens, const int32_t* __restrict__ parents, const int32_t* __restrict__ n_nodes,
    int nmax, int batch, int walk_step, int rows_by_batch, const uint32_t* __restrict__ noise, int noise_stride,
    int noise_col0, uint64_t seed, uint64_t step, const int32_t* __restrict__ seq_ids, int draw0, SampleParams sp,
    int32_t* acc_tokens, int32_t* acc_nodes, int acc_stride, int32_t* acc_len, int32_t* last_node,
    int32_t* correction, int32_t* state, int32_t* err_flag, int32_t* next_rows, int32_t* next_active) {
  __shared__ Shared sh;
  const int b = blockIdx.x;
  if (!state[batch + b]) return;
  const int parent = state[b];
  const int64_t slot = rows_by_batch ? (int64_t)b
                       : slot_map    ? (int64_t)slot_map[(int64_t)b * nmax + parent]
                                     : (int64_t)b * nmax + parent;
  if (slot < 0) {
    if (threadIdx.x == 0) {
      if (err_flag) atomicOr(err_flag, 2);
      state[batch + b] = 0;
      if (next_active) next_active[b] = 0;
    }
    return;
  }
  const char* rowp = (const char*)logits + slot * row_stride * (DT == fg::kBF16 ? 2 : 4);
  uint32_t seq = seq_ids ? (uint32_t)seq_ids[b] : (uint32_t)b;
  uint32_t u = noise_value(noise, (int64_t)b * noise_stride + noise_col0 + walk_step, seed, step, seq,
                           (uint32_t)(draw0 + walk_step));
  int tok = block_sample<DT>(rowp, vocab, sp, u, sh);
  if (threadIdx.x < 64)
    walk_apply(b, tok, parent, tree_tokens, parents, n_nodes, nmax, batch, walk_step, acc_tokens, acc_nodes, acc_stride,
               acc_len, last_node, correction, state, err_flag, next_rows, next_active);
}

// ------------------------------------------------------------------ split sampling
// Unrestricted draws (no top-k / top-p) and greedy draws spread one row over
// kSplitChunks workgroups instead of one. The row maximum and its first maximum
// come as parts: per-chunk parts of split_max_kernel, or the per-workgroup parts
// the LM head writes with the logits (fg_lm_head_topk's row maxima). Then (1) per
// chunk, the q-mass against the row maximum (split_sum_kernel); (2) per row, the
// chunk whose running mass crosses the target and the index inside it
// (split_pick_kernel) -- the same integer rule as block_sample, so the token is
// identical. Greedy draws need only the parts and the pick. The chunk sums are
// handed over at a launch boundary: a device-scope fence per workgroup to hand
// them over inside one launch measured slower than the second launch.
constexpr int kSplitChunks = 16;
constexpr int kSplitThreads = 256;
constexpr int kSplitWaves = kSplitThreads / 64;

struct SplitArgs {
  const void* logits;
  int64_t row_stride;
  int vocab;
  int chunk;                 // elements per chunk (multiple of 8)
  const int32_t* row_index;  // logits row of sampled row r (NULL: r)
  const int32_t* forced;     // rows with forced[r] >= 0 are not sampled
  const int32_t* active;     // rows with active[r] == 0 are not sampled (NULL: all)
  float temperature;
  int scale;
  int greedy;
  float* part_max;           // [rows, kSplitChunks]
  uint64_t* part_key;
  uint64_t* part_sum;
  uint64_t* part_gsum;       // [rows, kSplitChunks, kSplitMaxGroups] q-mass per group of kSplitGroup
  int groups;                // groups per chunk (group sums kept only up to kSplitMaxGroups)
  float* row_m;              // [rows] row maximum (sum launch -> pick launch)
  uint64_t* row_best;        // [rows] first maximum's rank key
  // row maxima parts read by the draw launch: [rows, src_stride], src_parts used
  const float* src_max;
  const uint64_t* src_key;
  int src_parts;
  int64_t src_stride;
  // split top-p (see "split top-p")
  uint32_t tp32;
  uint64_t* hist;            // [rows, kSplitChunks, 256] chunk histograms of one radix level
  struct SelState* sel;      // [rows, 2] select state, double-buffered across levels
  uint64_t* part_a;          // [rows, kSplitChunks] q-mass of keys above the cut key
  uint64_t* part_t;          // [rows, kSplitChunks] q-mass of keys equal to it
};

// Radix select state of one row: the selected key bits so far, the q-mass of
// keys above them, and the top-p target mass.
struct SelState {
  uint32_t prefix, pmask;
  uint64_t above, target;
};

template <int DT>
FG_DEVICE const char* split_row(const SplitArgs& a, int r) {
  const int64_t src = a.row_index ? a.row_index[r] : r;
  return (const char*)a.logits + src * a.row_stride * (DT == fg::kBF16 ? 2 : 4);
}

FG_DEVICE bool split_skip(const SplitArgs& a, int r) {
  return (a.forced && a.forced[r] >= 0) || (a.active && !a.active[r]);
}

// Elements per workgroup pass: kSplitLoads groups of 8 per thread, all loads in flight
// before the weights are computed (5 groups: a 152,064-logit row's 9,504-element chunk is
// one pass, so a chunk costs one memory round trip).
constexpr int kSplitLoads = 5;
constexpr int kSplitGroup = kSplitThreads * 8;
constexpr int kSplitPass = kSplitGroup * kSplitLoads;
// Per-group q-mass is kept for chunks of up to kSplitMaxGroups groups (vocabularies up to
// 16 x 16 x 2,048 = 524,288): the pick then weighs one group instead of the whole chunk.
constexpr int kSplitMaxGroups = 16;

// Load group u of a pass starting at base (elements base + (u * kSplitThreads + t) * 8 ..
// + 7 of thread t) holds an element before hi. Uniform over the workgroup: a group wholly
// past the chunk end is neither loaded nor weighed (a 9,504-element chunk is one full pass
// of 8,192 and one group of the second).
FG_DEVICE bool split_group_live(int base, int u, int hi) { return base + u * kSplitThreads * 8 < hi; }

// Loads elements i0 .. i0 + 7 of a chunk ending at hi; past hi come -inf, whose weight is
// 0 against any row maximum, so the weights need no per-element test.
template <int DT>
FG_DEVICE void split_load8(const char* p, int i0, int hi, float (&x)[8]) {
  if (i0 + 8 <= hi) {
    fg::load8<DT>(p, i0, x);
    return;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = i0 + j < hi ? fg::load_elem<DT>(p, i0 + j) : -INFINITY;
}

// Chunk maxima (raw maximum, NaN ignored, and the first-maximum rank key). Per pass a thread
// takes the maximum of its elements (NaN ignored) and then the first index holding it (the
// first NaN when there is one, which ranks highest), and forms one rank key per pass instead
// of one per element.
template <int DT>
__global__ void __launch_bounds__(kSplitThreads) split_max_kernel(SplitArgs a) {
  const int c = blockIdx.x, r = blockIdx.y;
  if (split_skip(a, r)) return;
  __shared__ float smax[kSplitWaves];
  __shared__ uint64_t skey[kSplitWaves];
  const char* p = split_row<DT>(a, r);
  const int lo = c * a.chunk, hi = min(a.vocab, lo + a.chunk);
  float mx = -INFINITY;
  uint64_t best = 0;
  for (int base = lo; base < hi; base += kSplitPass) {
    float x[kSplitLoads][8];
#pragma unroll
    for (int u = 0; u < kSplitLoads; ++u)
      if (split_group_live(base, u, hi)) split_load8<DT>(p, base + (u * kSplitThreads + threadIdx.x) * 8, hi, x[u]);
    // the -inf padding past hi never wins: real elements come first and the first index holding
    // the maximum is taken
    float pm = -INFINITY;
    bool nan = false;
#pragma unroll
    for (int u = 0; u < kSplitLoads; ++u) {
      if (!split_group_live(base, u, hi)) continue;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pm = fmaxf(pm, x[u][j]);
        nan |= x[u][j] != x[u][j];
      }
    }
    int first = -1;
    float kv = pm;
#pragma unroll
    for (int u = kSplitLoads - 1; u >= 0; --u) {
      if (!split_group_live(base, u, hi)) continue;
      const int i0 = base + (u * kSplitThreads + threadIdx.x) * 8;
#pragma unroll
      for (int j = 7; j >= 0; --j) first = (nan ? x[u][j] != x[u][j] : x[u][j] == pm) ? i0 + j : first;
    }
    if (nan) kv = __uint_as_float(0x7fc00000u);
    mx = fmaxf(mx, pm);
    if (first >= 0) {
      const uint64_t k = fg::rank_key(kv, (uint32_t)first);
      best = k > best ? k : best;
    }
  }
  mx = fg::wave_max(mx);
  best = fg::wave_max_u64(best);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    smax[wave] = mx;
    skey[wave] = best;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kSplitWaves; ++w) {
      mx = fmaxf(mx, smax[w]);
      best = skey[w] > best ? skey[w] : best;
    }
    a.part_max[r * kSplitChunks + c] = fmaxf(smax[0], mx);
    a.part_key[r * kSplitChunks + c] = skey[0] > best ? skey[0] : best;
  }
}

// Row maximum from the chunk maxima.
FG_DEVICE float split_row_max(const SplitArgs& a, int r) {
  float mx = -INFINITY;
  for (int c = 0; c < kSplitChunks; ++c) mx = fmaxf(mx, a.part_max[r * kSplitChunks + c]);
  return mx;
}

FG_DEVICE float split_kt(const SplitArgs& a) { return fg::weight_kt(a.scale != 0, a.temperature); }

FG_DEVICE uint64_t split_weight8(const float (&x)[8], float kt, float m, const uint64_t* tbl) {
  uint64_t acc = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) acc += fg::weight_q40(m, x[j], kt, tbl);
  return acc;
}

// Per row: the raw maximum and first maximum from the row's parts (whole block).
FG_DEVICE void split_parts_max(const SplitArgs& a, int r, float* smax, uint64_t* skey, float& mx, uint64_t& best) {
  const int tid = threadIdx.x;
  mx = -INFINITY;
  best = 0;
  for (int q = tid; q < a.src_parts; q += kSplitThreads) {
    mx = fmaxf(mx, a.src_max[r * a.src_stride + q]);
    const uint64_t k = a.src_key[r * a.src_stride + q];
    best = k > best ? k : best;
  }
  mx = fg::wave_max(mx);
  best = fg::wave_max_u64(best);
  if ((tid & 63) == 0) {
    smax[tid >> 6] = mx;
    skey[tid >> 6] = best;
  }
  __syncthreads();
  mx = smax[0];
  best = skey[0];
#pragma unroll
  for (int w = 1; w < kSplitWaves; ++w) {
    mx = fmaxf(mx, smax[w]);
    best = skey[w] > best ? skey[w] : best;
  }
}

// q-mass of each chunk against the row maximum taken from the row's parts; chunk 0 also
// keeps the scaled maximum and the first maximum for the pick launch.
template <int DT>
__global__ void __launch_bounds__(kSplitThreads) split_sum_kernel(SplitArgs a) {
  const int c = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
  if (split_skip(a, r)) return;
  __shared__ uint64_t tbl[1024];
  __shared__ float smax[kSplitWaves];
  __shared__ uint64_t skey[kSplitWaves];
  __shared__ uint64_t gsum[kSplitMaxGroups];
  const char* p = split_row<DT>(a, r);
  const int lo = c * a.chunk, hi = min(a.vocab, lo + a.chunk);
  // the first pass's logits are in flight while the row maximum is gathered from the parts
  float x[kSplitLoads][8];
#pragma unroll
  for (int u = 0; u < kSplitLoads; ++u)
    if (split_group_live(lo, u, hi)) split_load8<DT>(p, lo + (u * kSplitThreads + tid) * 8, hi, x[u]);
  fg::exp2_table_to_lds(tbl);  // visible after the barrier in split_parts_max
  if (tid < kSplitMaxGroups) gsum[tid] = 0;
  float mx;
  uint64_t best;
  split_parts_max(a, r, smax, skey, mx, best);
  const float m = mx, kt = split_kt(a);
  // each group's q-mass: wave sums added into LDS (group g of the chunk = elements
  // [lo + 2048 g, lo + 2048 (g + 1)) = load group u of pass g / 4)
  const bool keep_groups = a.groups <= kSplitMaxGroups;
  int g = 0;
  for (int base = lo; base < hi; base += kSplitPass) {
    if (base != lo) {
#pragma unroll
      for (int u = 0; u < kSplitLoads; ++u)
        if (split_group_live(base, u, hi)) split_load8<DT>(p, base + (u * kSplitThreads + tid) * 8, hi, x[u]);
    }
#pragma unroll
    for (int u = 0; u < kSplitLoads; ++u) {
      if (!split_group_live(base, u, hi)) continue;
      const uint64_t w = fg::wave_sum_u64(split_weight8(x[u], kt, m, tbl));
      if ((tid & 63) == 0) atomicAdd((unsigned long long*)&gsum[keep_groups ? g + u : 0], (unsigned long long)w);
    }
    g += kSplitLoads;
  }
  __syncthreads();
  if (tid == 0) {
    uint64_t t = 0;
    const int ng = keep_groups ? a.groups : 1;
    for (int q = 0; q < ng; ++q) {
      t += gsum[q];
      if (keep_groups) a.part_gsum[((size_t)r * kSplitChunks + c) * kSplitMaxGroups + q] = gsum[q];
    }
    a.part_sum[r * kSplitChunks + c] = t;
    if (c == 0) {
      a.row_m[r] = m;
      a.row_best[r] = best;
    }
  }
}

// First index in [lo, hi) whose inclusive running q-mass exceeds target (the whole
// block; -1 if none), scanned in index order one group of kSplitThreads x 8 elements at a
// time (thread t holds 8 consecutive elements of a group), stopping at the group that holds
// the target: on average half the chunk is weighed. A pass's groups are loaded together.
template <int DT>
FG_DEVICE int split_locate(const char* p, int lo, int hi, float m, float kt, const uint64_t* tbl, uint64_t target,
                           uint64_t* wsum, int* found) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) *found = -1;
  uint64_t run = 0;  // block-uniform
  bool done = false;
  for (int base = lo; base < hi && !done; base += kSplitPass) {
    float x[kSplitLoads][8];
#pragma unroll
    for (int u = 0; u < kSplitLoads; ++u)
      if (split_group_live(base, u, hi)) split_load8<DT>(p, base + (u * kSplitThreads + tid) * 8, hi, x[u]);
#pragma unroll
    for (int u = 0; u < kSplitLoads; ++u) {
      if (!split_group_live(base, u, hi)) break;  // uniform
      const uint64_t mine = split_weight8(x[u], kt, m, tbl);
      const uint64_t incl = fg::wave_incl_scan_u64(mine);
      __syncthreads();  // wsum of the previous group has been read
      if (lane == 63) wsum[wave] = incl;
      __syncthreads();
      uint64_t woff = 0, stot = 0;
#pragma unroll
      for (int w = 0; w < kSplitWaves; ++w) {
        if (w < wave) woff += wsum[w];
        stot += wsum[w];
      }
      if (run + stot > target) {  // uniform: this group holds the target
        uint64_t cum = run + woff + incl - mine;
        if (cum <= target && target < cum + mine) {
          const int i0 = base + (u * kSplitThreads + tid) * 8;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            cum += fg::weight_q40(m, x[u][j], kt, tbl);
            if (cum > target) {
              *found = i0 + j;
              break;
            }
          }
        }
        done = true;
        break;
      }
      run += stot;
    }
  }
  __syncthreads();
  return *found;
}

// Outputs of a draw: a token per row, or one step of the acceptance walk.
struct DrawOut {
  const uint32_t* noise;
  int noise_stride;
  int noise_col;   // walk: noise column noise_col + walk_step
  uint64_t seed, step;
  const int32_t* seq_ids;
  int draw;        // walk: counter draw draw + walk_step
  int32_t* out;    // [rows] (sample mode)
  // walk mode
  const int32_t* tree_tokens;
  const int32_t* parents;
  const int32_t* n_nodes;
  int nmax, batch, walk_step;
  int32_t* acc_tokens;
  int32_t* acc_nodes;
  int acc_stride;
  int32_t* acc_len;
  int32_t* last_node;
  int32_t* correction;
  int32_t* state;
  int32_t* err_flag;
  int32_t* next_rows;    // optional: the next walk step's LM-head rows
  int32_t* next_active;
};

// The draw of each row (one workgroup per row) from the chunk sums of split_sum_kernel
// (greedy draws: from the row's parts alone): the chunk whose running mass crosses the
// target, then the index inside it.
template <int DT, bool WALK>
__global__ void __launch_bounds__(kSplitThreads) split_pick_kernel(SplitArgs a, DrawOut d) {
  const int r = blockIdx.x, tid = threadIdx.x;
  __shared__ uint64_t tbl[1024];
  __shared__ float smax[kSplitWaves];
  __shared__ uint64_t skey[kSplitWaves];
  __shared__ uint64_t wsum[kSplitWaves];
  __shared__ int s_found;
  if constexpr (WALK) {
    if (!d.state[d.batch + r]) return;
  } else {
    if (a.forced && a.forced[r] >= 0) {
      if (tid == 0) d.out[r] = a.forced[r];
      return;
    }
  }
  int tok;
  if (a.greedy) {
    float mx;
    uint64_t best;
    split_parts_max(a, r, smax, skey, mx, best);
    tok = (int)fg::rank_key_index(best);
  } else {
    tok = (int)fg::rank_key_index(a.row_best[r]);
    uint64_t sums[kSplitChunks], total = 0;
#pragma unroll
    for (int q = 0; q < kSplitChunks; ++q) {
      sums[q] = a.part_sum[r * kSplitChunks + q];
      total += sums[q];
    }
    if (total > 0) {
      fg::exp2_table_to_lds(tbl);  // visible after split_locate's first barrier
      const uint32_t seq = d.seq_ids ? (uint32_t)d.seq_ids[r] : (uint32_t)r;
      const int ws = WALK ? d.walk_step : 0;
      const uint32_t u = noise_value(d.noise, (int64_t)r * d.noise_stride + d.noise_col + ws, d.seed, d.step, seq,
                                     (uint32_t)(d.draw + ws));
      const uint64_t target = fg::mulhi_u64_u32(total, u);
      uint64_t before = 0;
      int cs = kSplitChunks - 1;
      for (int q = 0; q < kSplitChunks; ++q) {
        if (before + sums[q] > target) {
          cs = q;
          break;
        }
        before += sums[q];
      }
      int clo = cs * a.chunk, chi = min(a.vocab, clo + a.chunk);
      if (a.groups <= kSplitMaxGroups) {
        // the group of 2,048 whose running mass crosses the target: one group is weighed
        const uint64_t* gs = a.part_gsum + ((size_t)r * kSplitChunks + cs) * kSplitMaxGroups;
        const int ng = (chi - clo + kSplitGroup - 1) / kSplitGroup;
        int q = ng - 1;
        for (int k = 0; k < ng; ++k) {
          if (before + gs[k] > target) {
            q = k;
            break;
          }
          before += gs[k];
        }
        clo += q * kSplitGroup;
        chi = min(chi, clo + kSplitGroup);
      }
      const int idx = split_locate<DT>(split_row<DT>(a, r), clo, chi, a.row_m[r], split_kt(a), tbl, target - before,
                                       wsum, &s_found);
      if (idx >= 0) tok = idx;  // always: the chunk holds the target
    }
  }
  if constexpr (WALK) {
    if (tid < 64)
      walk_apply(r, tok, d.state[r], d.tree_tokens, d.parents, d.n_nodes, d.nmax, d.batch, d.walk_step, d.acc_tokens,
                 d.acc_nodes, d.acc_stride, d.acc_len, d.last_node, d.correction, d.state, d.err_flag, d.next_rows,
                 d.next_active);
  } else {
    if (tid == 0) d.out[r] = tok;
  }
}

// ------------------------------------------------------------------ split top-p
// Top-p draws (no top-k) over kSplitChunks workgroups per row, the same integer
// rule as block_sample / radix_select: (1) chunk maxima (split_max_kernel);
// (2) four launches of one 8-bit radix level each over the scaled-logit keys: every
// chunk workgroup first merges the previous level's 16 chunk histograms (all of a
// row's workgroups reach the same digit; chunk 0 records the state) and then
// histograms its chunk's q-mass under the new prefix -- the first merge also yields
// the row's q total and the target floor(total * tp32 / 2^32); (3) the last merge
// fixes the cut key; each chunk sums the q-mass above it and tied with it;
// (4) one workgroup per row resolves the ties in index order, then locates the
// draw among the kept tokens in vocabulary order (chunk by chunk partial sums).

// Calls f(i, s, key) for the elements of chunk c of row r (8 per thread per step).
template <int DT, class F>
FG_DEVICE void for_chunk(const SplitArgs& a, int r, int c, F&& f) {
  const char* p = split_row<DT>(a, r);
  const int lo = c * a.chunk, hi = min(a.vocab, lo + a.chunk);
  for (int i0 = lo + threadIdx.x * 8; i0 < hi; i0 += kSplitThreads * 8) {
    float x[8];
    if (i0 + 8 <= hi) {
      fg::load8<DT>(p, i0, x);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = i0 + j < hi ? fg::load_elem<DT>(p, i0 + j) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (i0 + j < hi) {
        f(i0 + j, x[j], fg::sort_key32(x[j]));
      }
  }
}

// Sum of v over the workgroup (kSplitThreads threads).
FG_DEVICE uint64_t split_block_sum(uint64_t v, uint64_t* red) {
  v = fg::wave_sum_u64(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int w = 0; w < kSplitThreads / 64; ++w) t += red[w];
  return t;
}

// Merges the 16 chunk histograms of the level at `shift` into st (radix_select's
// digit rule); level 0's merge first sets the top-p target from the row total.
FG_DEVICE void split_merge_level(const SplitArgs& a, int r, int shift, bool first, SelState& st, uint64_t* hs,
                                 uint64_t* red, int* sdig, uint64_t* sabove) {
  const uint64_t* hp = a.hist + (size_t)r * kSplitChunks * 256;
  uint64_t v = 0;
  for (int c = 0; c < kSplitChunks; ++c) v += hp[c * 256 + threadIdx.x];
  hs[threadIdx.x] = v;
  if (first) st.target = fg::mulhi_u64_u32(split_block_sum(v, red), a.tp32);
  if (threadIdx.x == 0) {
    *sdig = 0;  // no digit holds the target only when the row total is 0 (then the draw is the argmax)
    *sabove = st.above;
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    uint64_t h[4], mine = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h[j] = hs[255 - 4 * lane - j];
      mine += h[j];
    }
    const uint64_t incl = fg::wave_incl_scan_u64(mine);
    const uint64_t excl = incl - mine;
    if (st.above + excl <= st.target && st.target < st.above + incl) {
      uint64_t c = st.above + excl;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (c + h[j] > st.target) {
          *sdig = 255 - 4 * lane - j;
          *sabove = c;
          break;
        }
        c += h[j];
      }
    }
  }
  __syncthreads();
  st.prefix |= (uint32_t)*sdig << shift;
  st.pmask |= 255u << shift;
  st.above = *sabove;
}

// One radix level (level 0..3, digit bits 31-8l .. 24-8l): merge the previous
// level, then this chunk's q-mass histogram under the prefix.
template <int DT>
__global__ void __launch_bounds__(kSplitThreads) split_topp_level_kernel(SplitArgs a, int level) {
  const int c = blockIdx.x, r = blockIdx.y;
  if (split_skip(a, r)) return;
  __shared__ uint64_t tbl[1024];
  __shared__ uint64_t hs[256];
  __shared__ uint64_t red[kSplitThreads / 64];
  __shared__ int sdig;
  __shared__ uint64_t sabove;
  fg::exp2_table_to_lds(tbl);  // visible after the barriers below
  SelState st{0u, 0u, 0ull, 0ull};
  if (level >= 2) st = a.sel[r * 2 + ((level - 2) & 1)];
  if (level >= 1) {
    split_merge_level(a, r, 24 - 8 * (level - 1), level == 1, st, hs, red, &sdig, &sabove);
    if (c == 0 && threadIdx.x == 0) a.sel[r * 2 + ((level - 1) & 1)] = st;
  }
  const float m = split_row_max(a, r), kt = split_kt(a);
  const int shift = 24 - 8 * level;
  __syncthreads();
  hs[threadIdx.x] = 0;
  __syncthreads();
  for_chunk<DT>(a, r, c, [&](int, float sv, uint32_t key) {
    if ((key & st.pmask) == st.prefix)
      atomicAdd((unsigned long long*)&hs[(key >> shift) & 255u],
                (unsigned long long)fg::weight_q40(m, sv, kt, tbl));
  });
  __syncthreads();
  a.hist[((size_t)r * kSplitChunks + c) * 256 + threadIdx.x] = hs[threadIdx.x];
}

// Last merge (the cut key), then this chunk's q-mass above the cut key and tied with it.
template <int DT>
__global__ void __launch_bounds__(kSplitThreads) split_topp_cut_kernel(SplitArgs a) {
  const int c = blockIdx.x, r = blockIdx.y;
  if (split_skip(a, r)) return;
  __shared__ uint64_t tbl[1024];
  __shared__ uint64_t hs[256];
  __shared__ uint64_t red[kSplitThreads / 64];
  __shared__ int sdig;
  __shared__ uint64_t sabove;
  fg::exp2_table_to_lds(tbl);  // visible after the barriers of the merge
  SelState st = a.sel[r * 2 + 0];  // after level 2
  split_merge_level(a, r, 0, false, st, hs, red, &sdig, &sabove);
  if (c == 0 && threadIdx.x == 0) a.sel[r * 2 + 1] = st;
  const float m = split_row_max(a, r), kt = split_kt(a);
  const uint32_t kappa = st.prefix;
  uint64_t above = 0, tie = 0;
  for_chunk<DT>(a, r, c, [&](int, float sv, uint32_t key) {
    if (key >= kappa) {
      const uint64_t w = fg::weight_q40(m, sv, kt, tbl);
      if (key > kappa) above += w;
      else tie += w;
    }
  });
  above = split_block_sum(above, red);
  tie = split_block_sum(tie, red);
  if (threadIdx.x == 0) {
    a.part_a[r * kSplitChunks + c] = above;
    a.part_t[r * kSplitChunks + c] = tie;
  }
}

// Chunk-relative predicates for the pick (element index i is relative to chunk start lo).
struct TieAt {
  uint32_t kappa;
  FG_DEVICE bool operator()(uint32_t key, uint32_t) const { return key == kappa; }
};
struct TieUpTo {
  uint32_t kappa, last_rel;
  FG_DEVICE bool operator()(uint32_t key, uint32_t i) const { return key == kappa && i <= last_rel; }
};
struct KeptIn {
  uint32_t kappa, last, lo;
  FG_DEVICE bool operator()(uint32_t key, uint32_t i) const { return key > kappa || (key == kappa && lo + i <= last); }
};

template <int DT>
FG_DEVICE Row<DT> chunk_row(const SplitArgs& a, int r, int c, const uint64_t* tbl) {
  const int lo = c * a.chunk;
  Row<DT> rr;
  rr.p = split_row<DT>(a, r) + (int64_t)lo * (DT == fg::kBF16 ? 2 : 4);
  rr.V = max(0, min(a.vocab, lo + a.chunk) - lo);
  rr.seg = (((rr.V + kWaves - 1) / kWaves) + kStep - 1) / kStep * kStep;
  rr.kt = split_kt(a);
  rr.tbl = tbl;
  rr.m = split_row_max(a, r);
  return rr;
}

// The token of row r (whole block; every thread returns it).
template <int DT>
FG_DEVICE int split_topp_pick(const SplitArgs& a, int r, uint32_t u, Shared& sh) {
  fg::exp2_table_to_lds(sh.exp2);  // visible after the first barrier of block_sum
  const SelState st = a.sel[r * 2 + 1];
  const uint32_t kappa = st.prefix;
  const uint64_t* pa = a.part_a + r * kSplitChunks;
  const uint64_t* pt = a.part_t + r * kSplitChunks;
  const uint64_t need = st.target - st.above;
  // ties on the cut key are kept in index order up to the one whose running mass exceeds `need`
  uint64_t tb = 0;
  int cs = -1;
  for (int c = 0; c < kSplitChunks; ++c) {
    if (tb + pt[c] > need) {
      cs = c;
      break;
    }
    tb += pt[c];
  }
  uint32_t last = 0xffffffffu;
  uint64_t tie_cs = 0;  // tie mass kept in chunk cs
  if (cs >= 0) {
    const Row<DT> rr = chunk_row<DT>(a, r, cs, sh.exp2);
    block_sum<true, DT>(rr, TieAt{kappa}, sh);
    const int idx = block_locate<true, DT>(rr, TieAt{kappa}, need - tb, sh);
    if (idx >= 0) {
      last = (uint32_t)(cs * a.chunk + idx);
      tie_cs = block_sum<true, DT>(rr, TieUpTo{kappa, (uint32_t)idx}, sh);
    } else {
      cs = -1;  // cannot happen: chunk cs holds the crossing tie
    }
  }
  uint64_t total = 0;
  for (int c = 0; c < kSplitChunks; ++c)
    total += pa[c] + (cs < 0 || c < cs ? pt[c] : (c == cs ? tie_cs : 0ull));
  uint64_t best = 0;
  for (int c = 0; c < kSplitChunks; ++c) {
    const uint64_t k = a.part_key[r * kSplitChunks + c];
    best = k > best ? k : best;
  }
  if (total == 0) return (int)fg::rank_key_index(best);
  const uint64_t target = fg::mulhi_u64_u32(total, u);
  uint64_t before = 0;
  int c2 = kSplitChunks - 1;
  for (int c = 0; c < kSplitChunks; ++c) {
    const uint64_t kc = pa[c] + (cs < 0 || c < cs ? pt[c] : (c == cs ? tie_cs : 0ull));
    if (before + kc > target) {
      c2 = c;
      break;
    }
    before += kc;
  }
  const Row<DT> r2 = chunk_row<DT>(a, r, c2, sh.exp2);
  const KeptIn kept{kappa, last, (uint32_t)(c2 * a.chunk)};
  block_sum<true, DT>(r2, kept, sh);
  const int idx = block_locate<true, DT>(r2, kept, target - before, sh);
  return idx >= 0 ? c2 * a.chunk + idx : (int)fg::rank_key_index(best);
}

template <int DT>
__global__ void __launch_bounds__(kThreads) split_topp_sample_kernel(SplitArgs a, const uint32_t* __restrict__ noise,
                                                                     int noise_stride, int noise_col, uint64_t seed,
                                                                     uint64_t step, const int32_t* __restrict__ seq_ids,
                                                                     int draw, int32_t* __restrict__ out) {
  __shared__ Shared sh;
  const int r = blockIdx.x;
  if (a.forced && a.forced[r] >= 0) {
    if (threadIdx.x == 0) out[r] = a.forced[r];
    return;
  }
  const uint32_t seq = seq_ids ? (uint32_t)seq_ids[r] : (uint32_t)r;
  const uint32_t u = noise_value(noise, (int64_t)r * noise_stride + noise_col, seed, step, seq, (uint32_t)draw);
  const int tok = split_topp_pick<DT>(a, r, u, sh);
  if (threadIdx.x == 0) out[r] = tok;
}

template <int DT>
__global__ void __launch_bounds__(kThreads) split_topp_walk_kernel(
    SplitArgs a, const int32_t* __restrict__ tree_tokens, const int32_t* __restrict__ parents,
    const int32_t* __restrict__ n_nodes, int nmax, int batch, int walk_step, const uint32_t* __restrict__ noise,
    int noise_stride, int noise_col0, uint64_t seed, uint64_t step, const int32_t* __restrict__ seq_ids, int draw0,
    int32_t* acc_tokens, int32_t* acc_nodes, int acc_stride, int32_t* acc_len, int32_t* last_node,
    int32_t* correction, int32_t* state, int32_t* err_flag, int32_t* next_rows, int32_t* next_active) {
  __shared__ Shared sh;
  const int b = blockIdx.x;
  if (!state[batch + b]) return;
  const int parent = state[b];
  const uint32_t seq = seq_ids ? (uint32_t)seq_ids[b] : (uint32_t)b;
  const uint32_t u = noise_value(noise, (int64_t)b * noise_stride + noise_col0 + walk_step, seed, step, seq,
                                 (uint32_t)(draw0 + walk_step));
  const int tok = split_topp_pick<DT>(a, b, u, sh);
  if (threadIdx.x < 64)
    walk_apply(b, tok, parent, tree_tokens, parents, n_nodes, nmax, batch, walk_step, acc_tokens, acc_nodes,
               acc_stride, acc_len, last_node, correction, state, err_flag, next_rows, next_active);
}

// Chunk partials of the split top-p path: max, four radix levels, the cut (6 launches).
template <int DT>
void split_topp_partials(const SplitArgs& a, int rows, hipStream_t s) {
  dim3 grid(kSplitChunks, rows);
  hipLaunchKernelGGL(split_max_kernel<DT>, grid, dim3(kSplitThreads), 0, s, a);
  for (int level = 0; level < 4; ++level)
    hipLaunchKernelGGL(split_topp_level_kernel<DT>, grid, dim3(kSplitThreads), 0, s, a, level);
  hipLaunchKernelGGL(split_topp_cut_kernel<DT>, grid, dim3(kSplitThreads), 0, s, a);
}

// A split draw: the chunk maxima unless a.src_* already hold row maxima parts, the
// chunk sums (not for greedy draws), the pick (1 to 3 launches).
template <int DT, bool WALK>
void split_draw(const SplitArgs& a, const DrawOut& d, int rows, bool with_max, hipStream_t s) {
  if (with_max) hipLaunchKernelGGL(split_max_kernel<DT>, dim3(kSplitChunks, rows), dim3(kSplitThreads), 0, s, a);
  if (!a.greedy) hipLaunchKernelGGL(split_sum_kernel<DT>, dim3(kSplitChunks, rows), dim3(kSplitThreads), 0, s, a);
  hipLaunchKernelGGL((split_pick_kernel<DT, WALK>), dim3(rows), dim3(kSplitThreads), 0, s, a, d);
}

constexpr size_t split_workspace_bytes(int rows) {
  return (size_t)rows * kSplitChunks * (4 + 8 + 8) + (size_t)rows * kSplitChunks * 256 * 8 +
         (size_t)rows * 2 * sizeof(SelState) + (size_t)rows * kSplitChunks * 16 + (size_t)rows * (8 + 4) +
         (size_t)rows * kSplitChunks * kSplitMaxGroups * 8 + 256;
}

// Scratch of fg_sample_tokens_noalloc: the split partials of up to
// kNoAllocMaxRows rows (9.1 MB per device, held until the process ends). Each
// kernel of the split paths writes every partial it owns before a later launch
// reads it, so nothing in it has to start at zero. Host code never hands
// `scratch` itself to a kernel (in host code the name is only a stand-in): it
// passes the per-device address that hipGetSymbolAddress returns.
constexpr int kNoAllocMaxRows = 256;
constexpr size_t kScratchBytes = split_workspace_bytes(kNoAllocMaxRows);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device.
int scratch_for_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fg::fail("fg_sample_tokens_noalloc: no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fg::fail(std::string("fg_sample_tokens_noalloc: hipGetSymbolAddress(scratch) failed: ") +
                      hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

// Carves the split partials out of a caller workspace; false when it is too small.
bool split_setup(SplitArgs& a, void* workspace, size_t bytes, int rows, const void* logits, int64_t row_stride,
                 int vocab, float temperature, int greedy) {
  if (!workspace || bytes < split_workspace_bytes(rows)) return false;
  char* w = (char*)(((uintptr_t)workspace + 15) & ~(uintptr_t)15);
  a.part_key = (uint64_t*)w;
  a.part_sum = a.part_key + (size_t)rows * kSplitChunks;
  a.hist = a.part_sum + (size_t)rows * kSplitChunks;
  a.part_a = a.hist + (size_t)rows * kSplitChunks * 256;
  a.part_t = a.part_a + (size_t)rows * kSplitChunks;
  a.sel = (SelState*)(a.part_t + (size_t)rows * kSplitChunks);
  a.row_best = (uint64_t*)(a.sel + (size_t)rows * 2);
  a.part_gsum = a.row_best + rows;
  a.part_max = (float*)(a.part_gsum + (size_t)rows * kSplitChunks * kSplitMaxGroups);
  a.row_m = a.part_max + (size_t)rows * kSplitChunks;
  a.src_max = a.part_max;
  a.src_key = a.part_key;
  a.src_parts = kSplitChunks;
  a.src_stride = kSplitChunks;
  a.tp32 = 0;
  a.logits = logits;
  a.row_stride = row_stride;
  a.vocab = vocab;
  a.chunk = ((vocab + kSplitChunks - 1) / kSplitChunks + 7) / 8 * 8;
  a.groups = (a.chunk + kSplitGroup - 1) / kSplitGroup;
  a.temperature = temperature;
  a.greedy = greedy || temperature == 0.0f;
  a.scale = !a.greedy && temperature > 0.0f && temperature != 1.0f;
  a.row_index = nullptr;
  a.forced = nullptr;
  a.active = nullptr;
  return true;
}

// Length clamp, EOS cut, finished flag and the b200 pending root.
// Follows flashgrpo/decoding/flash_medusa_decoder.py:899-922 and
// flashgrpo_b200/decoding/flash_medusa_decoder.py:2303-2319.
__global__ void accept_finalize_kernel(const int32_t* __restrict__ acc_tokens, const int32_t* __restrict__ acc_nodes,
                                       int acc_stride, int32_t* acc_len, int32_t* last_node,
                                       const int32_t* __restrict__ correction, const int32_t* __restrict__ old_len,
                                       int max_length, int eos_token_id, int32_t* finished, int32_t* pending_root,
                                       int batch) {
  int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const int raw = acc_len[b];
  int keep = max(1, max_length - old_len[b]);
  int len = min(raw, keep);
  int eos = 0;
  if (eos_token_id >= 0) {
    for (int j = 0; j < len; ++j)
      if (acc_tokens[(int64_t)b * acc_stride + j] == eos_token_id) {
        len = j + 1;
        eos = 1;
        break;
      }
  }
  acc_len[b] = len;
  last_node[b] = acc_nodes[(int64_t)b * acc_stride + len - 1];
  int fin = eos || old_len[b] + len >= max_length;
  finished[b] = fin;
  if (pending_root) pending_root[b] = (correction[b] >= 0 && len == raw && !fin) ? correction[b] : -1;
}

SampleParams make_params(float temperature, int greedy, int top_k, int vocab, uint32_t tp32) {
  SampleParams sp;
  sp.temperature = temperature;
  sp.greedy = greedy || temperature == 0.0f;
  sp.top_k = (top_k > 0 && top_k < vocab) ? top_k : 0;
  sp.tp32 = tp32;
  return sp;
}

int sample_tokens_impl(const char* who, const void* logits, int dtype, int64_t row_stride, int rows, int vocab,
                       const int32_t* row_index, const int32_t* forced, const uint32_t* noise,
                       int noise_stride, int noise_col, uint64_t seed, uint64_t step,
                       const int32_t* seq_ids, int draw, float temperature, int greedy, int top_k,
                       uint32_t top_p_fixed, int32_t* out_tokens, void* workspace,
                       size_t workspace_bytes, void* stream) {
  FG_REQUIRE(logits && out_tokens, std::string(who) + ": null pointer");
  FG_REQUIRE(rows > 0 && vocab > 0 && vocab < (1 << 23), std::string(who) + ": vocab must be in [1, 2^23)");
  FG_REQUIRE(dtype == fg::kF32 || dtype == fg::kBF16, std::string(who) + ": dtype");
  FG_REQUIRE(row_stride >= vocab && row_stride % 8 == 0 && ((uintptr_t)logits & 31) == 0,
             std::string(who) + ": rows must be 32-byte aligned (row_stride % 8 == 0)");
  SampleParams sp = make_params(temperature, greedy, top_k, vocab, top_p_fixed);
  hipStream_t s = (hipStream_t)stream;
  SplitArgs a;
  if ((sp.greedy || (sp.top_k == 0 && sp.tp32 == 0)) &&
      split_setup(a, workspace, workspace_bytes, rows, logits, row_stride, vocab, temperature, sp.greedy)) {
    a.row_index = row_index;
    a.forced = forced;
    DrawOut d{};
    d.noise = noise; d.noise_stride = noise_stride; d.noise_col = noise_col;
    d.seed = seed; d.step = step; d.seq_ids = seq_ids; d.draw = draw; d.out = out_tokens;
    if (dtype == fg::kBF16) split_draw<fg::kBF16, false>(a, d, rows, true, s);
    else split_draw<fg::kF32, false>(a, d, rows, true, s);
    return fg::check_launch(who);
  }
  if (!sp.greedy && sp.top_k == 0 && sp.tp32 != 0 &&
      split_setup(a, workspace, workspace_bytes, rows, logits, row_stride, vocab, temperature, 0)) {
    a.row_index = row_index;
    a.forced = forced;
    a.tp32 = sp.tp32;
    if (dtype == fg::kBF16) {
      split_topp_partials<fg::kBF16>(a, rows, s);
      hipLaunchKernelGGL(split_topp_sample_kernel<fg::kBF16>, dim3(rows), dim3(kThreads), 0, s, a, noise,
                         noise_stride, noise_col, seed, step, seq_ids, draw, out_tokens);
    } else {
      split_topp_partials<fg::kF32>(a, rows, s);
      hipLaunchKernelGGL(split_topp_sample_kernel<fg::kF32>, dim3(rows), dim3(kThreads), 0, s, a, noise,
                         noise_stride, noise_col, seed, step, seq_ids, draw, out_tokens);
    }
    return fg::check_launch(who);
  }
  if (dtype == fg::kBF16)
    hipLaunchKernelGGL(sample_rows_kernel<fg::kBF16>, dim3(rows), dim3(kThreads), 0, s, logits, row_stride, vocab,
                       row_index, forced, noise, noise_stride, noise_col, seed, step, seq_ids, draw, sp, out_tokens);
  else
    hipLaunchKernelGGL(sample_rows_kernel<fg::kF32>, dim3(rows), dim3(kThreads), 0, s, logits, row_stride, vocab,
                       row_index, forced, noise, noise_stride, noise_col, seed, step, seq_ids, draw, sp, out_tokens);
  return fg::check_launch(who);
}

}  // namespace

extern "C" {

size_t fg_sample_workspace(int rows) { return rows > 0 ? split_workspace_bytes(rows) : 0; }

int fg_sample_tokens(const void* logits, int dtype, int64_t row_stride, int rows, int vocab,
                     const int32_t* row_index, const int32_t* forced, const uint32_t* noise, int noise_stride,
                     int noise_col, uint64_t seed, uint64_t step, const int32_t* seq_ids, int draw,
                     float temperature, int greedy, int top_k, uint32_t top_p_fixed, int32_t* out_tokens,
                     void* workspace, size_t workspace_bytes, void* stream) {
  return sample_tokens_impl("fg_sample_tokens", logits, dtype, row_stride, rows, vocab, row_index, forced, noise,
                            noise_stride, noise_col, seed, step, seq_ids, draw, temperature, greedy, top_k,
                            top_p_fixed, out_tokens, workspace, workspace_bytes, stream);
}

size_t fg_sample_tokens_noalloc_max_rows(void) { return kNoAllocMaxRows; }

int fg_sample_tokens_noalloc(const void* logits, int dtype, int64_t row_stride, int rows, int vocab,
                             const int32_t* row_index, const int32_t* forced, const uint32_t* noise,
                             int noise_stride, int noise_col, uint64_t seed, uint64_t step, const int32_t* seq_ids,
                             int draw, float temperature, int greedy, int top_k, uint32_t top_p_fixed,
                             int32_t* out_tokens, void* stream) {
  FG_REQUIRE(rows > 0 && rows <= kNoAllocMaxRows,
             "fg_sample_tokens_noalloc: rows must be in [1, " + std::to_string(kNoAllocMaxRows) + "] (got " +
                 std::to_string(rows) + ")");
  void* ws = nullptr;
  if (int rc = scratch_for_current_device(&ws)) return rc;
  return sample_tokens_impl("fg_sample_tokens_noalloc", logits, dtype, row_stride, rows, vocab, row_index, forced,
                            noise, noise_stride, noise_col, seed, step, seq_ids, draw, temperature, greedy, top_k,
                            top_p_fixed, out_tokens, ws, kScratchBytes, stream);
}

int fg_accept_walk(const void* tree_logits, int dtype, int64_t row_stride, int vocab, const int32_t* slot_map,
                   const int32_t* tree_tokens, const int32_t* parents, const int32_t* n_nodes, int nmax, int batch,
                   int max_walk_steps, const uint32_t* noise, int noise_stride, int noise_col0, uint64_t seed,
                   uint64_t step, const int32_t* seq_ids, int draw0, float temperature, int greedy, int top_k,
                   uint32_t top_p_fixed, int32_t* acc_tokens, int32_t* acc_nodes, int acc_stride, int32_t* acc_len,
                   int32_t* last_node, int32_t* correction, int32_t* workspace, int32_t* err_flag, void* stream) {
  FG_REQUIRE(tree_logits && tree_tokens && parents && n_nodes && acc_tokens && acc_nodes && acc_len && last_node &&
                 correction && workspace,
             "fg_accept_walk: null pointer");
  FG_REQUIRE(batch > 0 && nmax > 0 && nmax <= 64 && vocab > 0 && vocab < (1 << 23), "fg_accept_walk: bad shape");
  FG_REQUIRE(acc_stride >= 1 && max_walk_steps >= 0, "fg_accept_walk: bad acc_stride / steps");
  FG_REQUIRE(dtype == fg::kF32 || dtype == fg::kBF16, "fg_accept_walk: dtype");
  FG_REQUIRE(row_stride >= vocab && row_stride % 8 == 0 && ((uintptr_t)tree_logits & 31) == 0,
             "fg_accept_walk: rows must be 32-byte aligned (row_stride % 8 == 0)");
  SampleParams sp = make_params(temperature, greedy, top_k, vocab, top_p_fixed);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(walk_init_kernel, dim3((batch + 63) / 64), dim3(64), 0, s, tree_tokens, parents, n_nodes, nmax,
                     batch, acc_tokens, acc_nodes, acc_stride, acc_len, last_node, correction, workspace);
  for (int t = 0; t < max_walk_steps; ++t) {
    if (dtype == fg::kBF16)
      hipLaunchKernelGGL(walk_step_kernel<fg::kBF16>, dim3(batch), dim3(kThreads), 0, s, tree_logits, row_stride,
                         vocab, slot_map, tree_tokens, parents, n_nodes, nmax, batch, t, 0, noise, noise_stride,
                         noise_col0, seed, step, seq_ids, draw0, sp, acc_tokens, acc_nodes, acc_stride, acc_len,
                         last_node, correction, workspace, err_flag, nullptr, nullptr);
    else
      hipLaunchKernelGGL(walk_step_kernel<fg::kF32>, dim3(batch), dim3(kThreads), 0, s, tree_logits, row_stride,
                         vocab, slot_map, tree_tokens, parents, n_nodes, nmax, batch, t, 0, noise, noise_stride,
                         noise_col0, seed, step, seq_ids, draw0, sp, acc_tokens, acc_nodes, acc_stride, acc_len,
                         last_node, correction, workspace, err_flag, nullptr, nullptr);
  }
  return fg::check_launch("fg_accept_walk");
}

int fg_walk_begin(const int32_t* tree_tokens, const int32_t* parents, const int32_t* n_nodes, int nmax, int batch,
                  int32_t* acc_tokens, int32_t* acc_nodes, int acc_stride, int32_t* acc_len, int32_t* last_node,
                  int32_t* correction, int32_t* state, void* stream) {
  FG_REQUIRE(tree_tokens && parents && n_nodes && acc_tokens && acc_nodes && acc_len && last_node && correction &&
                 state,
             "fg_walk_begin: null pointer");
  FG_REQUIRE(batch > 0 && nmax > 0 && nmax <= 64 && acc_stride >= 1, "fg_walk_begin: bad shape");
  hipLaunchKernelGGL(walk_init_kernel, dim3((batch + 63) / 64), dim3(64), 0, (hipStream_t)stream, tree_tokens,
                     parents, n_nodes, nmax, batch, acc_tokens, acc_nodes, acc_stride, acc_len, last_node, correction,
                     state);
  return fg::check_launch("fg_walk_begin");
}

int fg_walk_rows(const int32_t* state, int batch, int nmax, int32_t* row_index, int32_t* row_active, void* stream) {
  FG_REQUIRE(state && row_index && row_active && batch > 0 && nmax > 0, "fg_walk_rows: bad arguments");
  hipLaunchKernelGGL(walk_rows_kernel, dim3((batch + 63) / 64), dim3(64), 0, (hipStream_t)stream, state, batch, nmax,
                     row_index, row_active);
  return fg::check_launch("fg_walk_rows");
}

int fg_walk_step(const void* step_logits, int dtype, int64_t row_stride, int vocab, const int32_t* tree_tokens,
                 const int32_t* parents, const int32_t* n_nodes, int nmax, int batch, int walk_step,
                 const uint32_t* noise, int noise_stride, int noise_col0, uint64_t seed, uint64_t step,
                 const int32_t* seq_ids, int draw0, float temperature, int greedy, int top_k, uint32_t top_p_fixed,
                 int32_t* acc_tokens, int32_t* acc_nodes, int acc_stride, int32_t* acc_len, int32_t* last_node,
                 int32_t* correction, int32_t* state, int32_t* err_flag, const float* part_max,
                 const uint64_t* part_key, int nparts, int32_t* next_row_index, int32_t* next_row_active,
                 void* workspace, size_t workspace_bytes, void* stream) {
  FG_REQUIRE(step_logits && tree_tokens && parents && n_nodes && acc_tokens && acc_nodes && acc_len && last_node &&
                 correction && state,
             "fg_walk_step: null pointer");
  FG_REQUIRE(batch > 0 && nmax > 0 && nmax <= 64 && vocab > 0 && vocab < (1 << 23) && walk_step >= 0,
             "fg_walk_step: bad shape");
  FG_REQUIRE(dtype == fg::kF32 || dtype == fg::kBF16, "fg_walk_step: dtype");
  FG_REQUIRE(row_stride >= vocab && row_stride % 8 == 0 && ((uintptr_t)step_logits & 31) == 0,
             "fg_walk_step: rows must be 32-byte aligned (row_stride % 8 == 0)");
  FG_REQUIRE(!part_max == !part_key && (!part_max || nparts > 0), "fg_walk_step: part_max / part_key / nparts");
  FG_REQUIRE(!next_row_index == !next_row_active, "fg_walk_step: next_row_index and next_row_active go together");
  SampleParams sp = make_params(temperature, greedy, top_k, vocab, top_p_fixed);
  hipStream_t s = (hipStream_t)stream;
  SplitArgs a;
  if ((sp.greedy || (sp.top_k == 0 && sp.tp32 == 0)) &&
      split_setup(a, workspace, workspace_bytes, batch, step_logits, row_stride, vocab, temperature, sp.greedy)) {
    a.active = state + batch;
    const bool with_max = part_max == nullptr;
    if (!with_max) {
      a.src_max = part_max;
      a.src_key = part_key;
      a.src_parts = nparts;
      a.src_stride = nparts;
    }
    DrawOut d{};
    d.noise = noise; d.noise_stride = noise_stride; d.noise_col = noise_col0;
    d.seed = seed; d.step = step; d.seq_ids = seq_ids; d.draw = draw0;
    d.tree_tokens = tree_tokens; d.parents = parents; d.n_nodes = n_nodes;
    d.nmax = nmax; d.batch = batch; d.walk_step = walk_step;
    d.acc_tokens = acc_tokens; d.acc_nodes = acc_nodes; d.acc_stride = acc_stride; d.acc_len = acc_len;
    d.last_node = last_node; d.correction = correction; d.state = state; d.err_flag = err_flag;
    d.next_rows = next_row_index; d.next_active = next_row_active;
    if (dtype == fg::kBF16) split_draw<fg::kBF16, true>(a, d, batch, with_max, s);
    else split_draw<fg::kF32, true>(a, d, batch, with_max, s);
    return fg::check_launch("fg_walk_step");
  }
  if (!sp.greedy && sp.top_k == 0 && sp.tp32 != 0 &&
      split_setup(a, workspace, workspace_bytes, batch, step_logits, row_stride, vocab, temperature, 0)) {
    a.active = state + batch;
    a.tp32 = sp.tp32;
    if (dtype == fg::kBF16) {
      split_topp_partials<fg::kBF16>(a, batch, s);
      hipLaunchKernelGGL(split_topp_walk_kernel<fg::kBF16>, dim3(batch), dim3(kThreads), 0, s, a, tree_tokens, parents,
                         n_nodes, nmax, batch, walk_step, noise, noise_stride, noise_col0, seed, step, seq_ids, draw0,
                         acc_tokens, acc_nodes, acc_stride, acc_len, last_node, correction, state, err_flag,
                         next_row_index, next_row_active);
    } else {
      split_topp_partials<fg::kF32>(a, batch, s);
      hipLaunchKernelGGL(split_topp_walk_kernel<fg::kF32>, dim3(batch), dim3(kThreads), 0, s, a, tree_tokens, parents,
                         n_nodes, nmax, batch, walk_step, noise, noise_stride, noise_col0, seed, step, seq_ids, draw0,
                         acc_tokens, acc_nodes, acc_stride, acc_len, last_node, correction, state, err_flag,
                         next_row_index, next_row_active);
    }
    return fg::check_launch("fg_walk_step");
  }
  if (dtype == fg::kBF16)
    hipLaunchKernelGGL(walk_step_kernel<fg::kBF16>, dim3(batch), dim3(kThreads), 0, s, step_logits, row_stride, vocab,
                       nullptr, tree_tokens, parents, n_nodes, nmax, batch, walk_step, 1, noise, noise_stride,
                       noise_col0, seed, step, seq_ids, draw0, sp, acc_tokens, acc_nodes, acc_stride, acc_len,
                       last_node, correction, state, err_flag, next_row_index, next_row_active);
  else
    hipLaunchKernelGGL(walk_step_kernel<fg::kF32>, dim3(batch), dim3(kThreads), 0, s, step_logits, row_stride, vocab,
                       nullptr, tree_tokens, parents, n_nodes, nmax, batch, walk_step, 1, noise, noise_stride,
                       noise_col0, seed, step, seq_ids, draw0, sp, acc_tokens, acc_nodes, acc_stride, acc_len,
                       last_node, correction, state, err_flag, next_row_index, next_row_active);
  return fg::check_launch("fg_walk_step");
}

int fg_accept_finalize(const int32_t* acc_tokens, const int32_t* acc_nodes, int acc_stride, int32_t* acc_len,
                       int32_t* last_node, const int32_t* correction, const int32_t* old_len, int max_length,
                       int eos_token_id, int32_t* finished, int32_t* pending_root, int batch, void* stream) {
  FG_REQUIRE(acc_tokens && acc_nodes && acc_len && last_node && correction && old_len && finished,
             "fg_accept_finalize: null pointer");
  FG_REQUIRE(batch > 0 && acc_stride >= 1, "fg_accept_finalize: bad shape");
  hipLaunchKernelGGL(accept_finalize_kernel, dim3((batch + 63) / 64), dim3(64), 0, (hipStream_t)stream, acc_tokens,
                     acc_nodes, acc_stride, acc_len, last_node, correction, old_len, max_length, eos_token_id,
                     finished, pending_root, batch);
  return fg::check_launch("fg_accept_finalize");
}

}  // extern "C"
