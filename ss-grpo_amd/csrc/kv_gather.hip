// Accepted-path KV compaction (all layers, K and V, one launch).
//
// For every sequence b the accepted nodes' cache rows seq_len[b] + node[j]
// move to seq_len[b] + j, j < acc_len[b]. Destinations overlap sources
// (node[j] >= j), so each workgroup first stages every source row of its
// (tensor, sequence) in LDS, then writes: the copy has the read-all-then-write
// semantics of the reference's gather(...).contiguous() + copy_
// (flashgrpo/decoding/kv_extraction.py:54-84).
#include "fg_common.h"

namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads) kv_path_gather_kernel(
    const uint64_t* __restrict__ tensor_ptrs, int kv_heads, int row_bytes, int64_t batch_stride_b,
    int64_t head_stride_b, int64_t row_stride_b, int capacity, const int32_t* __restrict__ seq_len,
    const int32_t* __restrict__ row_map, const int32_t* __restrict__ acc_nodes, int acc_stride,
    const int32_t* __restrict__ acc_len, int tree_nodes, int32_t* __restrict__ err_flag) {
  extern __shared__ uint4 stage[];
  const int t = blockIdx.x;  // tensor (K or V of one layer)
  const int b = blockIdx.y;  // sequence
  const int n_acc = acc_len[b];
  const int s0 = seq_len[b];
  // Validate the whole row before touching memory.
  bool ok = n_acc >= 1 && n_acc <= acc_stride && s0 >= 0 && s0 + tree_nodes <= capacity;
  for (int j = 0; j < n_acc && ok; ++j) {
    int nd = acc_nodes[(int64_t)b * acc_stride + j];
    ok = nd >= 0 && nd < tree_nodes;
  }
  if (!ok) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, 1);
    return;
  }
  const int cb = row_map ? row_map[b] : b;
  char* base = (char*)(uintptr_t)tensor_ptrs[t] + (int64_t)cb * batch_stride_b;
  const int chunks_per_row = row_bytes >> 4;
  const int total = kv_heads * n_acc * chunks_per_row;
  for (int c = threadIdx.x; c < total; c += kThreads) {
    int col = c % chunks_per_row;
    int r = c / chunks_per_row;
    int j = r % n_acc;
    int h = r / n_acc;
    int nd = acc_nodes[(int64_t)b * acc_stride + j];
    const uint4* src = (const uint4*)(base + h * head_stride_b + (int64_t)(s0 + nd) * row_stride_b) + col;
    stage[c] = *src;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < total; c += kThreads) {
    int col = c % chunks_per_row;
    int r = c / chunks_per_row;
    int j = r % n_acc;
    int h = r / n_acc;
    uint4* dst = (uint4*)(base + h * head_stride_b + (int64_t)(s0 + j) * row_stride_b) + col;
    *dst = stage[c];
  }
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
  const size_t lds = (size_t)kv_heads * acc_stride * row_bytes;
  FG_REQUIRE(lds <= 64 * 1024, "fg_kv_path_gather: kv_heads*acc_stride*row_bytes exceeds 64 KiB");
  dim3 grid(num_tensors, batch);
  hipLaunchKernelGGL(kv_path_gather_kernel, grid, dim3(kThreads), lds, (hipStream_t)stream, tensor_ptrs, kv_heads,
                     row_bytes, batch_stride * elem_bytes, head_stride * elem_bytes, row_stride * elem_bytes,
                     capacity, seq_len, row_map, acc_nodes, acc_stride, acc_len, tree_nodes, err_flag);
  return fg::check_launch("fg_kv_path_gather");
}
