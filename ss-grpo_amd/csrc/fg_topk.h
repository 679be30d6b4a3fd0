// Top-k list helpers shared by the per-row top-k kernels (topk.hip) and the LM-head
// epilogue (lm_head.hip). Lists hold 64-bit rank keys (fg::rank_key: value desc, index
// asc) sorted descending; 0 is the empty slot and ranks below every key.
#pragma once

#include "fg_common.h"

#include <cmath>

namespace fg {

template <int K>
FG_DEVICE void insert_key(uint64_t (&top)[K], uint64_t k) {
  if (k <= top[K - 1]) return;
  top[K - 1] = k;
#pragma unroll
  for (int i = K - 1; i > 0; --i) {
    if (top[i] > top[i - 1]) {
      uint64_t t = top[i];
      top[i] = top[i - 1];
      top[i - 1] = t;
    }
  }
}

// Sort a bitonic sequence of K keys into descending order.
template <int K>
FG_DEVICE void bitonic_sort_desc(uint64_t (&v)[K]) {
#pragma unroll
  for (int len = K / 2; len > 0; len >>= 1) {
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if ((i & len) == 0) {
        int j = i | len;
        if (v[j] > v[i]) {
          uint64_t t = v[i];
          v[i] = v[j];
          v[j] = t;
        }
      }
    }
  }
}

// top-K of two descending lists, result descending in `a`.
template <int K>
FG_DEVICE void merge_desc(uint64_t (&a)[K], const uint64_t (&b)[K]) {
#pragma unroll
  for (int i = 0; i < K; ++i) {
    uint64_t o = b[K - 1 - i];
    a[i] = o > a[i] ? o : a[i];
  }
  bitonic_sort_desc<K>(a);
}

// Merge the lists within each group of `lanes` consecutive lanes (a power of two <= 64);
// every lane of a group ends with the group's list.
template <int K>
FG_DEVICE void lanes_merge(uint64_t (&top)[K], int lanes) {
  for (int o = lanes / 2; o > 0; o >>= 1) {
    uint64_t other[K];
#pragma unroll
    for (int i = 0; i < K; ++i) other[i] = shfl_xor_u64(top[i], o);
    merge_desc<K>(top, other);
  }
}

template <int K>
FG_DEVICE void wave_merge(uint64_t (&top)[K]) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t other[K];
#pragma unroll
    for (int i = 0; i < K; ++i) other[i] = shfl_xor_u64(top[i], o);
    merge_desc<K>(top, other);
  }
}

// torch.nan_to_num(x, nan=-1e9, posinf=1e9, neginf=-1e9) when SAN.
template <bool SAN>
FG_DEVICE float sanitize(float v) {
  if constexpr (SAN) {
    if (v != v) return -1.0e9f;
    if (v == INFINITY) return 1.0e9f;
    if (v == -INFINITY) return -1.0e9f;
  }
  return v;
}

// Running (max, sum of exp(x - max)) of a set of values.
struct LseAcc {
  float m, s;
};

FG_DEVICE LseAcc lse_combine(LseAcc a, LseAcc b) {
  float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return {m, 0.0f};
  return {m, a.s * __expf(a.m - m) + b.s * __expf(b.m - m)};
}

// Merge per-part lists into each row's top-kout (cand_tokens / cand_scores [rows, kout])
// and, when row_stats is given, its (max, logsumexp) [rows, 2]. part_keys
// [rows, nparts, K] (K in {1, 2, 4, 8, 16}), part_lse [rows, nparts].
int topk_merge_parts(int K, const uint64_t* part_keys, const float2* part_lse, int rows, int nparts, int kout,
                     int32_t* cand_tokens, float* cand_scores, float* row_stats, hipStream_t stream);

}  // namespace fg
