// Accepted-path KV compaction (all layers, K and V, one launch).
//
// For every sequence b the accepted nodes' cache rows seq_len[b] + node[j]
// move to seq_len[b] + j, j < acc_len[b]. Destinations overlap sources, so the
// copy keeps the read-all-then-write semantics of the reference's
// gather(...).contiguous() + copy_ (flashgrpo/decoding/kv_extraction.py:54-84):
// one thread owns one 16-byte column of one (tensor, sequence, kv head) and
// loads all its accepted source chunks into registers before storing any, and
// no two threads touch the same column. Rows that stay in place (node[j] == j,
// always the root) are neither read nor written.
#include "fg_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxAcc = 32;  // longest accepted path (registers per thread)

template <int MAXACC>
__global__ void __launch_bounds__(kThreads) kv_path_gather_kernel(
    const uint64_t* __restrict__ tensor_ptrs, int batch, int kv_heads, int chunks_per_row, int total,
    int64_t batch_stride_b, int64_t head_stride_b, int64_t row_stride_b, int capacity,
    const int32_t* __restrict__ seq_len, const int32_t* __restrict__ row_map, const int32_t* __restrict__ acc_nodes,
    int acc_stride, const int32_t* __restrict__ acc_len, int tree_nodes, int32_t* __restrict__ err_flag) {
  const int gid = blockIdx.x * kThreads + threadIdx.x;  // total < 2^31 (host check)
  if (gid >= total) return;
  // gid = ((t * batch + b) * kv_heads + h) * chunks_per_row + col: consecutive threads walk one row
  const int col = gid % chunks_per_row;
  int r = gid / chunks_per_row;
  const int h = r % kv_heads;
  r /= kv_heads;
  const int b = r % batch;
  const int t = r / batch;
  const int32_t* nodes = acc_nodes + (int64_t)b * acc_stride;
  // Every per-sequence value is loaded in one round trip (the path entries up to the row
  // stride, independent of its length), then the whole row is validated before touching
  // the caches.
  const int n_acc = acc_len[b];
  const int s0 = seq_len[b];
  const int cb = row_map ? row_map[b] : b;
  const uint64_t tptr = tensor_ptrs[t];
  int nd[MAXACC];
#pragma unroll
  for (int j = 0; j < MAXACC; ++j) nd[j] = j < acc_stride ? nodes[j] : j;
  bool ok = n_acc >= 1 && n_acc <= acc_stride && n_acc <= tree_nodes && s0 >= 0 && s0 + tree_nodes <= capacity;
#pragma unroll
  for (int j = 0; j < MAXACC; ++j) {
    ok &= j >= n_acc || (nd[j] >= 0 && nd[j] < tree_nodes);
    nd[j] = j < n_acc ? nd[j] : j;
  }
  if (!ok) {
    if (t == 0 && h == 0 && col == 0 && err_flag) atomicOr(err_flag, 1);
    return;
  }
  char* base = (char*)(uintptr_t)tptr + (int64_t)cb * batch_stride_b + (int64_t)h * head_stride_b +
               (int64_t)col * 16 + (int64_t)s0 * row_stride_b;
  uint4 v[MAXACC];
#pragma unroll
  for (int j = 0; j < MAXACC; ++j)
    v[j] = nd[j] != j ? *(const uint4*)(base + (int64_t)nd[j] * row_stride_b) : make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < MAXACC; ++j)
    if (nd[j] != j) *(uint4*)(base + (int64_t)j * row_stride_b) = v[j];
}

}  // namespace

extern "C" int fg_kv_path_gather(const uint64_t* tensor_ptrs, int num_tensors, int batch, int kv_heads,
                                 int head_dim, int elem_bytes, int64_t batch_stride, int64_t head_stride,
                                 int64_t row_stride, int capacity, const int32_t* seq_len,
                                 const int32_t* row_map, const int32_t* acc_nodes, int acc_stride,
                                 const int32_t* acc_len, int tree_nodes, int32_t* err_flag, void* stream) {
  FG_REQUIRE(tensor_ptrs && seq_len && acc_nodes && acc_len, "fg_kv_path_gather: null pointer");
  FG_REQUIRE(num_tensors > 0 && batch > 0 && kv_heads > 0 && head_dim > 0, "fg_kv_path_gather: empty shape");
  FG_REQUIRE(elem_bytes == 2 || elem_bytes == 4, "fg_kv_path_gather: elem_bytes must be 2 or 4");
  const int row_bytes = head_dim * elem_bytes;
  FG_REQUIRE(row_bytes % 16 == 0, "fg_kv_path_gather: head_dim*elem_bytes must be a multiple of 16");
  FG_REQUIRE(acc_stride >= 1 && tree_nodes >= 1 && capacity >= tree_nodes, "fg_kv_path_gather: bad sizes");
  FG_REQUIRE((row_stride * elem_bytes) % 16 == 0 && (head_stride * elem_bytes) % 16 == 0 &&
                 (batch_stride * elem_bytes) % 16 == 0,
             "fg_kv_path_gather: strides must keep 16-byte alignment");
  FG_REQUIRE(acc_stride <= kMaxAcc, "fg_kv_path_gather: acc_stride (accepted path length) must be at most 32");
  const int chunks_per_row = row_bytes / 16;
  const int64_t total = (int64_t)num_tensors * batch * kv_heads * chunks_per_row;
  FG_REQUIRE(total < (1ll << 31) - kThreads, "fg_kv_path_gather: too many rows for one launch");
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  auto kern = acc_stride <= 8 ? kv_path_gather_kernel<8> : kv_path_gather_kernel<kMaxAcc>;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream,
                     tensor_ptrs, batch, kv_heads, chunks_per_row, (int)total, batch_stride * elem_bytes,
                     head_stride * elem_bytes, row_stride * elem_bytes, capacity, seq_len, row_map, acc_nodes,
                     acc_stride, acc_len, tree_nodes, err_flag);
  return fg::check_launch("fg_kv_path_gather");
}
