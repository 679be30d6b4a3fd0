// Per-token pieces of the verify forward around the projections: rotary
// embedding fused with the tree K/V slot write, RMSNorm (optionally fused with
// the residual add) and the SwiGLU gate. These mirror the Qwen2/Llama decoder
// layer that the reference runs through transformers
// (flashgrpo/models/qwen_flashgrpo_wrapper.py:172-180).
#include "fg_common.h"

namespace {

// One workgroup per token (b, n). qkv row = [q heads | k heads | v heads] x d.
// Position = seq_len[b] + pos_offset[n]; cache slot = seq_len[b] + n.
template <int DT>
__global__ void __launch_bounds__(256) rope_kv_write_kernel(
    const void* __restrict__ qkv, int64_t ld_qkv, int N, int Hq, int Hkv, int d, const int32_t* __restrict__ seq_len,
    const int32_t* __restrict__ pos_offset, const float* __restrict__ inv_freq, void* __restrict__ q_out,
    void* __restrict__ k_cache, void* __restrict__ v_cache, int64_t cache_batch, int64_t cache_head, int capacity,
    const int32_t* __restrict__ row_map, int32_t* __restrict__ err_flag) {
  const int tok = blockIdx.x;
  const int b = tok / N, n = tok % N;
  const int s = seq_len[b];
  const int pos = s + pos_offset[n];
  const int slot = s + n;
  const int cb = row_map ? row_map[b] : b;
  const int half = d / 2;
  const bool slot_ok = slot >= 0 && slot < capacity;
  if (!slot_ok && threadIdx.x == 0 && err_flag) atomicOr(err_flag, 8);
  const int64_t row = (int64_t)tok * ld_qkv;
  // q and k heads: rotate pairs (i, i + d/2)
  for (int e = threadIdx.x; e < (Hq + Hkv) * half; e += blockDim.x) {
    int h = e / half, i = e % half;
    float ang = (float)pos * inv_freq[i];
    float c = cosf(ang), sn = sinf(ang);
    int64_t src = row + (int64_t)h * d;
    float x1 = fg::load_elem<DT>(qkv, src + i);
    float x2 = fg::load_elem<DT>(qkv, src + i + half);
    float y1 = x1 * c - x2 * sn;
    float y2 = x2 * c + x1 * sn;
    if (h < Hq) {
      int64_t dst = ((int64_t)tok * Hq + h) * d;
      fg::store_elem<DT>(q_out, dst + i, y1);
      fg::store_elem<DT>(q_out, dst + i + half, y2);
    } else if (slot_ok) {
      int hk = h - Hq;
      int64_t dst = (int64_t)cb * cache_batch + (int64_t)hk * cache_head + (int64_t)slot * d;
      fg::store_elem<DT>(k_cache, dst + i, y1);
      fg::store_elem<DT>(k_cache, dst + i + half, y2);
    }
  }
  for (int e = threadIdx.x; slot_ok && e < Hkv * d; e += blockDim.x) {
    int hk = e / d, i = e % d;
    float x = fg::load_elem<DT>(qkv, row + (int64_t)(Hq + Hkv + hk) * d + i);
    fg::store_elem<DT>(v_cache, (int64_t)cb * cache_batch + (int64_t)hk * cache_head + (int64_t)slot * d + i, x);
  }
}

// y = RMSNorm(x [+ delta]) * w; with delta the sum is written back to x first.
template <int DT>
__global__ void __launch_bounds__(256) rmsnorm_kernel(void* __restrict__ x, const void* __restrict__ delta,
                                                      const void* __restrict__ w, void* __restrict__ y, int H,
                                                      float eps) {
  const int64_t base = (int64_t)blockIdx.x * H;
  __shared__ float red[4];
  float ss = 0.0f;
  for (int i = threadIdx.x; i < H; i += 256) {
    float v = fg::load_elem<DT>(x, base + i);
    if (delta) {
      v += fg::load_elem<DT>(delta, base + i);
      fg::store_elem<DT>(x, base + i, v);
      v = fg::load_elem<DT>(x, base + i);  // the stored (rounded) residual feeds the norm
    }
    ss += v * v;
  }
  ss = fg::wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float rs = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)H + eps);
  for (int i = threadIdx.x; i < H; i += 256) {
    float v = fg::load_elem<DT>(x, base + i);
    fg::store_elem<DT>(y, base + i, v * rs * fg::load_elem<DT>(w, i));
  }
}

// out[t, i] = silu(gu[t, i]) * gu[t, F + i]
template <int DT>
__global__ void swiglu_kernel(const void* __restrict__ gu, void* __restrict__ out, int F, int64_t total) {
  int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  int64_t t = e / F, i = e % F;
  float gt = fg::load_elem<DT>(gu, t * 2 * F + i);
  float up = fg::load_elem<DT>(gu, t * 2 * F + F + i);
  fg::store_elem<DT>(out, e, gt / (1.0f + __expf(-gt)) * up);
}

}  // namespace

extern "C" {

int fg_rope_kv_write(const void* qkv, int dtype, int64_t ld_qkv, int batch, int num_nodes, int q_heads, int kv_heads,
                     int head_dim, const int32_t* seq_len, const int32_t* pos_offset, const float* inv_freq,
                     void* q_out, void* k_cache, void* v_cache, int64_t cache_batch_stride,
                     int64_t cache_head_stride, int capacity, const int32_t* row_map, int32_t* err_flag,
                     void* stream) {
  FG_REQUIRE(qkv && seq_len && pos_offset && inv_freq && q_out && k_cache && v_cache, "fg_rope_kv_write: null pointer");
  FG_REQUIRE(batch > 0 && num_nodes > 0 && q_heads > 0 && kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0,
             "fg_rope_kv_write: bad shape");
  hipStream_t s = (hipStream_t)stream;
  dim3 grid(batch * num_nodes);
  if (dtype == fg::kBF16)
    hipLaunchKernelGGL(rope_kv_write_kernel<fg::kBF16>, grid, dim3(256), 0, s, qkv, ld_qkv, num_nodes, q_heads,
                       kv_heads, head_dim, seq_len, pos_offset, inv_freq, q_out, k_cache, v_cache,
                       cache_batch_stride, cache_head_stride, capacity, row_map, err_flag);
  else
    hipLaunchKernelGGL(rope_kv_write_kernel<fg::kF32>, grid, dim3(256), 0, s, qkv, ld_qkv, num_nodes, q_heads,
                       kv_heads, head_dim, seq_len, pos_offset, inv_freq, q_out, k_cache, v_cache,
                       cache_batch_stride, cache_head_stride, capacity, row_map, err_flag);
  return fg::check_launch("fg_rope_kv_write");
}

int fg_rmsnorm(void* x, const void* delta, const void* weight, void* y, int dtype, int rows, int hidden, float eps,
               void* stream) {
  FG_REQUIRE(x && weight && y && rows > 0 && hidden > 0, "fg_rmsnorm: bad arguments");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == fg::kBF16)
    hipLaunchKernelGGL(rmsnorm_kernel<fg::kBF16>, dim3(rows), dim3(256), 0, s, x, delta, weight, y, hidden, eps);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<fg::kF32>, dim3(rows), dim3(256), 0, s, x, delta, weight, y, hidden, eps);
  return fg::check_launch("fg_rmsnorm");
}

int fg_swiglu(const void* gate_up, void* out, int dtype, int rows, int inter, void* stream) {
  FG_REQUIRE(gate_up && out && rows > 0 && inter > 0, "fg_swiglu: bad arguments");
  int64_t total = (int64_t)rows * inter;
  dim3 grid((unsigned)((total + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == fg::kBF16)
    hipLaunchKernelGGL(swiglu_kernel<fg::kBF16>, grid, dim3(256), 0, s, gate_up, out, inter, total);
  else
    hipLaunchKernelGGL(swiglu_kernel<fg::kF32>, grid, dim3(256), 0, s, gate_up, out, inter, total);
  return fg::check_launch("fg_swiglu");
}

}  // extern "C"
