// Per-token pieces of the verify forward around the projections: rotary
// embedding fused with the tree K/V slot write, RMSNorm (optionally fused with
// the residual add) and the SwiGLU gate. These mirror the Qwen2/Llama decoder
// layer that the reference runs through transformers
// (flashgrpo/models/qwen_flashgrpo_wrapper.py:172-180). Also the chain proposals'
// ChainDraftCell input normalisation (flashgrpo/models/medusa_heads.py:12-42).
#include "fg_common.h"

namespace {

// A value rounded to the row dtype (bf16: round to nearest even; fp32: itself). The
// explicit roundings below keep the rounding points of the Hugging Face modules (and the
// rotary products are not contracted into FMAs, so fp32 rows round them too).
template <int DT>
FG_DEVICE float rnd(float x) {
  if constexpr (DT == fg::kBF16)
    return fg::round_bf16(x);
  else
    return x;
}

// 4 consecutive elements as floats (8 bytes bf16 / 16 bytes fp32).
template <int DT>
FG_DEVICE void load4(const void* p, int64_t i, float (&v)[4]) {
  if constexpr (DT == fg::kBF16) {
    uint2 r = *(const uint2*)((const uint16_t*)p + i);
    v[0] = __uint_as_float(r.x << 16);
    v[1] = __uint_as_float(r.x & 0xffff0000u);
    v[2] = __uint_as_float(r.y << 16);
    v[3] = __uint_as_float(r.y & 0xffff0000u);
  } else {
    float4 a = *(const float4*)((const float*)p + i);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  }
}

template <int DT>
FG_DEVICE void store4(void* p, int64_t i, const float (&v)[4]) {
  if constexpr (DT == fg::kBF16)
    *(uint2*)((uint16_t*)p + i) = make_uint2(fg::pack_bf16x2(v[0], v[1]), fg::pack_bf16x2(v[2], v[3]));
  else
    *(float4*)((float*)p + i) = make_float4(v[0], v[1], v[2], v[3]);
}

// Where rope_kv_write_kernel reads a token's projected qkv row: a row of the qkv tensor
// (PARTS false), or the fp32 split-K partial sums of the projection (fg_linear_parts, row stride
// ld = the projection's width) summed in split order, plus the bias, rounded to the row dtype as the
// projection's output would be (PARTS true).
template <int DT, bool PARTS>
struct QkvSource {
  const void* qkv;
  const float* part;
  int64_t part_stride;
  int splits;
  const void* bias;

  FG_DEVICE void get4(int64_t row, int col, float (&v)[4]) const {
    if constexpr (!PARTS) {
      load4<DT>(qkv, row + col, v);
      return;
    }
    const float* src = part + row + col;
    float4 a = *(const float4*)src;
    for (int s = 1; s < splits; ++s) {
      const float4 b = *(const float4*)(src + s * part_stride);
      a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
    }
    float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (bias) load4<DT>(bias, col, bv);
    v[0] = rnd<DT>(a.x + bv[0]);
    v[1] = rnd<DT>(a.y + bv[1]);
    v[2] = rnd<DT>(a.z + bv[2]);
    v[3] = rnd<DT>(a.w + bv[3]);
  }

  FG_DEVICE void get8(int64_t row, int col, float (&v)[8]) const {
    if constexpr (!PARTS) {
      fg::load8<DT>(qkv, row + col, v);
    } else {
      float lo[4], hi[4];
      get4(row, col, lo);
      get4(row, col + 4, hi);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = lo[j];
        v[4 + j] = hi[j];
      }
    }
  }
};

// One workgroup per token (b, n). qkv row = [q heads | k heads | v heads] x d.
// Position = seq_len[b] + pos_offset[b * pos_stride + n]; cache slot = seq_len[b] + n.
// cos/sin of the token's d/2 angles are computed once into LDS; each thread then
// rotates 4 consecutive pairs (i, i + d/2) of one head with 8/16-byte accesses.
// Requires d % 8 == 0 and d <= 256.
template <int DT, bool PARTS>
__global__ void __launch_bounds__(256) rope_kv_write_kernel(
    QkvSource<DT, PARTS> qkv, int64_t ld_qkv, int N, int Hq, int Hkv, int d, const int32_t* __restrict__ seq_len,
    const int32_t* __restrict__ pos_offset, int64_t pos_stride, const float* __restrict__ inv_freq,
    void* __restrict__ q_out,
    void* __restrict__ k_cache, void* __restrict__ v_cache, int64_t cache_batch, int64_t cache_head, int capacity,
    const int32_t* __restrict__ row_map, int32_t* __restrict__ err_flag) {
  __shared__ float cs[128], sn[128];
  const int tok = blockIdx.x;
  const int b = tok / N, n = tok % N;
  const int s = seq_len[b];
  const int pos = s + pos_offset[(int64_t)b * pos_stride + n];
  const int slot = s + n;
  const int cb = row_map ? row_map[b] : b;
  const int half = d / 2;
  const bool slot_ok = slot >= 0 && slot < capacity;
  if (!slot_ok && threadIdx.x == 0 && err_flag) atomicOr(err_flag, 8);
  for (int i = threadIdx.x; i < half; i += blockDim.x) {
    const float ang = (float)pos * inv_freq[i];
    cs[i] = rnd<DT>(cosf(ang));  // the HF rotary embedding casts cos / sin to the model dtype
    sn[i] = rnd<DT>(sinf(ang));
  }
  __syncthreads();
  const int64_t row = (int64_t)tok * ld_qkv;
  const int quads = half / 4;
  // q and k heads: rotate pairs (i, i + d/2), 4 pairs per item
  for (int e = threadIdx.x; e < (Hq + Hkv) * quads; e += blockDim.x) {
    const int h = e / quads, i0 = (e % quads) * 4;
    float x1[4], x2[4], y1[4], y2[4];
    qkv.get4(row, h * d + i0, x1);
    qkv.get4(row, h * d + i0 + half, x2);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma clang fp contract(off)
      // q * cos + rotate_half(q) * sin, each product and the sum rounded to the row dtype
      const float c = cs[i0 + j], sv = sn[i0 + j];
      y1[j] = rnd<DT>(rnd<DT>(x1[j] * c) - rnd<DT>(x2[j] * sv));
      y2[j] = rnd<DT>(rnd<DT>(x2[j] * c) + rnd<DT>(x1[j] * sv));
    }
    if (h < Hq) {
      const int64_t dst = ((int64_t)tok * Hq + h) * d;
      store4<DT>(q_out, dst + i0, y1);
      store4<DT>(q_out, dst + i0 + half, y2);
    } else if (slot_ok) {
      const int64_t dst = (int64_t)cb * cache_batch + (int64_t)(h - Hq) * cache_head + (int64_t)slot * d;
      store4<DT>(k_cache, dst + i0, y1);
      store4<DT>(k_cache, dst + i0 + half, y2);
    }
  }
  const int oct = d / 8;
  for (int e = threadIdx.x; slot_ok && e < Hkv * oct; e += blockDim.x) {
    const int hk = e / oct, i0 = (e % oct) * 8;
    float x[8];
    qkv.get8(row, (Hq + Hkv + hk) * d + i0, x);
    fg::store8<DT>(v_cache, (int64_t)cb * cache_batch + (int64_t)hk * cache_head + (int64_t)slot * d + i0, x);
  }
}

// y = RMSNorm(x [+ delta]) * w; with delta the sum is written back to x first and
// the stored (rounded) residual feeds the norm. One workgroup per row, 8
// elements per access; the row stays in registers between the two passes.
// Requires H % 8 == 0 and H <= 8 * 256 * kNormChunks.
constexpr int kNormChunks = 4;

template <int DT>
__global__ void __launch_bounds__(256) rmsnorm_kernel(void* __restrict__ x, const void* __restrict__ delta,
                                                      const void* __restrict__ w, void* __restrict__ y, int H,
                                                      float eps) {
  const int64_t base = (int64_t)blockIdx.x * H;
  const int nch = H / 8;
  __shared__ float red[4];
  float v[kNormChunks][8];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int ch = threadIdx.x + c * 256;
    if (ch < nch) {
      fg::load8<DT>(x, base + ch * 8, v[c]);
      if (delta) {
        float dv[8];
        fg::load8<DT>(delta, base + ch * 8, dv);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[c][j] += dv[j];
        fg::store8<DT>(x, base + ch * 8, v[c]);
        if constexpr (DT == fg::kBF16) {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[c][j] = fg::bf16_to_f32(fg::f32_to_bf16(v[c][j]));
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += v[c][j] * v[c][j];
    }
  }
  ss = fg::wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float rs = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)H + eps);
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int ch = threadIdx.x + c * 256;
    if (ch < nch) {
      float wv[8], o[8];
      fg::load8<DT>(w, ch * 8, wv);
      // x * rsqrt(mean x^2 + eps) rounded to the row dtype, then times the weight (the HF
      // RMSNorm's order)
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = wv[j] * rnd<DT>(v[c][j] * rs);
      fg::store8<DT>(y, base + ch * 8, o);
    }
  }
}

// out[t, i] = silu(gu[t, i]) * gu[t, F + i]; 8 elements per thread over a flat grid of
// rows x F/8 chunks (a grid row per token left the last workgroup of each row partly idle:
// 34.8 against 33.2 µs at the Qwen2.5-7B shape). Requires F % 8 == 0. In bf16, SiLU(gate) is
// rounded to bf16 before the product, as the Hugging Face MLP computes act_fn(gate) * up under
// bf16 autocast.
FG_DEVICE float silu_in(float g, int dt) {
  const float s = fg::silu_f32(g);
  return dt == fg::kBF16 ? fg::round_bf16(s) : s;
}

template <int DT>
__global__ void __launch_bounds__(256) swiglu_kernel(const void* __restrict__ gu, void* __restrict__ out, int F,
                                                     int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int chunks = F / 8;
  const int64_t t = i / chunks;
  const int ch = (int)(i - t * chunks);
  float g[8], u[8], o[8];
  fg::load8<DT>(gu, t * 2 * F + ch * 8, g);
  fg::load8<DT>(gu, t * 2 * F + F + ch * 8, u);
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = silu_in(g[j], DT) * u[j];
  fg::store8<DT>(out, t * F + ch * 8, o);
}

// The ChainDraftCell's two normalised inputs side by side: workgroup (r, 0) writes
// out[r, 0:H] = LayerNorm(state[r]) * sw + sb and (r, 1) out[r, H:2H] = LayerNorm(token[r]) * tw + tb
// (mean, then the mean squared deviation, over the row held in registers; fp32 math, affine
// weights in the row dtype). H % 8 == 0, H <= 8192.
template <int DT>
__global__ void __launch_bounds__(256) chain_cell_norm_kernel(const void* __restrict__ state, int64_t lds_,
                                                              const void* __restrict__ token, int64_t ldt,
                                                              const void* __restrict__ sw, const void* __restrict__ sb,
                                                              const void* __restrict__ tw, const void* __restrict__ tb,
                                                              int H, float eps, void* __restrict__ out) {
  const int r = blockIdx.x, which = blockIdx.y, tid = threadIdx.x;
  const void* src = which ? token : state;
  const int64_t base = (int64_t)r * (which ? ldt : lds_);
  const void* w = which ? tw : sw;
  const void* bb = which ? tb : sb;
  const int nch = H / 8;
  __shared__ float red[8];
  float v[kNormChunks][8];
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int ch = tid + c * 256;
    if (ch < nch) {
      fg::load8<DT>(src, base + ch * 8, v[c]);
#pragma unroll
      for (int j = 0; j < 8; ++j) s += v[c][j];
    }
  }
  s = fg::wave_sum(s);
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  const float mean = (red[0] + red[1] + red[2] + red[3]) / (float)H;
  float q = 0.0f;
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c)
    if (tid + c * 256 < nch) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float d = v[c][j] - mean;
        q += d * d;
      }
    }
  q = fg::wave_sum(q);
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = q;
  __syncthreads();
  const float rstd = rsqrtf((red[4] + red[5] + red[6] + red[7]) / (float)H + eps);
  const int64_t obase = (int64_t)r * 2 * H + (int64_t)which * H;
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int ch = tid + c * 256;
    if (ch < nch) {
      float wv[8], bv[8], y[8];
      fg::load8<DT>(w, ch * 8, wv);
      fg::load8<DT>(bb, ch * 8, bv);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = (v[c][j] - mean) * rstd * wv[j] + bv[j];
      fg::store8<DT>(out, obase + ch * 8, y);
    }
  }
}

}  // namespace

extern "C" {

}  // extern "C"

namespace {

int rope_kv_write_launch(const char* what, const void* qkv, const float* part, int64_t part_stride, int splits,
                         const void* bias, int dtype, int64_t ld_qkv, int batch, int num_nodes, int q_heads,
                         int kv_heads, int head_dim, const int32_t* seq_len, const int32_t* pos_offset,
                         int64_t pos_batch_stride, const float* inv_freq, void* q_out, void* k_cache, void* v_cache,
                         int64_t cache_batch_stride, int64_t cache_head_stride, int capacity, const int32_t* row_map,
                         int32_t* err_flag, void* stream) {
  const std::string w(what);
  FG_REQUIRE((qkv || part) && seq_len && pos_offset && inv_freq && q_out && k_cache && v_cache, w + ": null pointer");
  FG_REQUIRE(batch > 0 && num_nodes > 0 && q_heads > 0 && kv_heads > 0, w + ": bad shape");
  FG_REQUIRE(pos_batch_stride == 0 || pos_batch_stride >= num_nodes, w + ": pos_batch_stride must be 0 or >= num_nodes");
  FG_REQUIRE(head_dim > 0 && head_dim % 8 == 0 && head_dim <= 256, w + ": head_dim must be a multiple of 8 in [8, 256]");
  FG_REQUIRE(ld_qkv % 8 == 0 && ((uintptr_t)qkv & 15) == 0 && ((uintptr_t)part & 15) == 0 &&
                 ((uintptr_t)bias & 15) == 0 && ((uintptr_t)q_out & 15) == 0 && ((uintptr_t)k_cache & 15) == 0 &&
                 ((uintptr_t)v_cache & 15) == 0 && cache_batch_stride % 8 == 0 && cache_head_stride % 8 == 0,
             w + ": rows must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  dim3 grid(batch * num_nodes);
#define FG_ROPE(DTv, PARTSv)                                                                                     \
  {                                                                                                              \
    const QkvSource<DTv, PARTSv> src{qkv, part, part_stride, splits, bias};                                      \
    hipLaunchKernelGGL((rope_kv_write_kernel<DTv, PARTSv>), grid, dim3(256), 0, s, src, ld_qkv, num_nodes, q_heads, \
                       kv_heads, head_dim, seq_len, pos_offset, pos_batch_stride, inv_freq, q_out, k_cache, v_cache, \
                       cache_batch_stride, cache_head_stride, capacity, row_map, err_flag);                       \
  }
  if (dtype == fg::kBF16 && part) FG_ROPE(fg::kBF16, true)
  else if (dtype == fg::kBF16) FG_ROPE(fg::kBF16, false)
  else if (part) FG_ROPE(fg::kF32, true)
  else FG_ROPE(fg::kF32, false)
#undef FG_ROPE
  return fg::check_launch(what);
}

}  // namespace

extern "C" {

int fg_rope_kv_write(const void* qkv, int dtype, int64_t ld_qkv, int batch, int num_nodes, int q_heads, int kv_heads,
                     int head_dim, const int32_t* seq_len, const int32_t* pos_offset, int64_t pos_batch_stride,
                     const float* inv_freq, void* q_out, void* k_cache, void* v_cache, int64_t cache_batch_stride,
                     int64_t cache_head_stride, int capacity, const int32_t* row_map, int32_t* err_flag,
                     void* stream) {
  FG_REQUIRE(qkv, "fg_rope_kv_write: null pointer");
  return rope_kv_write_launch("fg_rope_kv_write", qkv, nullptr, 0, 1, nullptr, dtype, ld_qkv, batch, num_nodes,
                              q_heads, kv_heads, head_dim, seq_len, pos_offset, pos_batch_stride, inv_freq, q_out,
                              k_cache, v_cache, cache_batch_stride, cache_head_stride, capacity, row_map, err_flag,
                              stream);
}

int fg_rope_kv_write_parts(const float* part, int splits, const void* bias, int dtype, int batch, int num_nodes,
                           int q_heads, int kv_heads, int head_dim, const int32_t* seq_len, const int32_t* pos_offset,
                           int64_t pos_batch_stride, const float* inv_freq, void* q_out, void* k_cache, void* v_cache,
                           int64_t cache_batch_stride, int64_t cache_head_stride, int capacity,
                           const int32_t* row_map, int32_t* err_flag, void* stream) {
  FG_REQUIRE(part && splits >= 1, "fg_rope_kv_write_parts: part must be given with splits >= 1");
  FG_REQUIRE(batch > 0 && num_nodes > 0 && q_heads > 0 && kv_heads > 0 && head_dim > 0,
             "fg_rope_kv_write_parts: bad shape");
  const int64_t width = (int64_t)(q_heads + 2 * kv_heads) * head_dim;
  return rope_kv_write_launch("fg_rope_kv_write_parts", nullptr, part, (int64_t)batch * num_nodes * width, splits, bias,
                              dtype, width, batch, num_nodes, q_heads, kv_heads, head_dim, seq_len, pos_offset,
                              pos_batch_stride, inv_freq, q_out, k_cache, v_cache, cache_batch_stride,
                              cache_head_stride, capacity, row_map, err_flag, stream);
}

int fg_rmsnorm(void* x, const void* delta, const void* weight, void* y, int dtype, int rows, int hidden, float eps,
               void* stream) {
  FG_REQUIRE(x && weight && y && rows > 0 && hidden > 0, "fg_rmsnorm: bad arguments");
  FG_REQUIRE(hidden % 8 == 0 && hidden <= 8 * 256 * kNormChunks, "fg_rmsnorm: hidden must be a multiple of 8, at most 8192");
  FG_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)weight & 15) == 0 && ((uintptr_t)y & 15) == 0 &&
                 (!delta || ((uintptr_t)delta & 15) == 0),
             "fg_rmsnorm: 16-byte alignment");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == fg::kBF16)
    hipLaunchKernelGGL(rmsnorm_kernel<fg::kBF16>, dim3(rows), dim3(256), 0, s, x, delta, weight, y, hidden, eps);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<fg::kF32>, dim3(rows), dim3(256), 0, s, x, delta, weight, y, hidden, eps);
  return fg::check_launch("fg_rmsnorm");
}

int fg_chain_cell_norm(const void* state, int64_t ld_state, const void* token, int64_t ld_token, int dtype,
                       int rows, int hidden, const void* state_w, const void* state_b, const void* token_w,
                       const void* token_b, float eps, void* out, void* stream) {
  FG_REQUIRE(state && token && state_w && state_b && token_w && token_b && out, "fg_chain_cell_norm: null pointer");
  FG_REQUIRE(dtype == fg::kBF16 || dtype == fg::kF32, "fg_chain_cell_norm: dtype");
  FG_REQUIRE(rows > 0 && rows <= 65535 && hidden > 0, "fg_chain_cell_norm: bad shape");
  FG_REQUIRE(hidden % 8 == 0 && hidden <= 8 * 256 * kNormChunks, "fg_chain_cell_norm: hidden must be a multiple of 8, at most 8192");
  FG_REQUIRE(ld_state >= hidden && ld_token >= hidden && ld_state % 8 == 0 && ld_token % 8 == 0,
             "fg_chain_cell_norm: row strides must be multiples of 8, at least hidden");
  const uintptr_t al = (uintptr_t)state | (uintptr_t)token | (uintptr_t)state_w | (uintptr_t)state_b |
                       (uintptr_t)token_w | (uintptr_t)token_b | (uintptr_t)out;
  FG_REQUIRE((al & 15) == 0, "fg_chain_cell_norm: 16-byte alignment");
  const dim3 grid((unsigned)rows, 2);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == fg::kBF16)
    hipLaunchKernelGGL(chain_cell_norm_kernel<fg::kBF16>, grid, dim3(256), 0, s, state, ld_state, token, ld_token,
                       state_w, state_b, token_w, token_b, hidden, eps, out);
  else
    hipLaunchKernelGGL(chain_cell_norm_kernel<fg::kF32>, grid, dim3(256), 0, s, state, ld_state, token, ld_token,
                       state_w, state_b, token_w, token_b, hidden, eps, out);
  return fg::check_launch("fg_chain_cell_norm");
}

int fg_swiglu(const void* gate_up, void* out, int dtype, int rows, int inter, void* stream) {
  FG_REQUIRE(gate_up && out && rows > 0 && inter > 0, "fg_swiglu: bad arguments");
  FG_REQUIRE(inter % 8 == 0 && ((uintptr_t)gate_up & 15) == 0 && ((uintptr_t)out & 15) == 0,
             "fg_swiglu: intermediate size must be a multiple of 8 with 16-byte aligned rows");
  const int64_t total = (int64_t)rows * (inter / 8);
  FG_REQUIRE((total + 255) / 256 < (1ll << 31), "fg_swiglu: too many rows for one call");
  const dim3 grid((unsigned)((total + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == fg::kBF16)
    hipLaunchKernelGGL(swiglu_kernel<fg::kBF16>, grid, dim3(256), 0, s, gate_up, out, inter, total);
  else
    hipLaunchKernelGGL(swiglu_kernel<fg::kF32>, grid, dim3(256), 0, s, gate_up, out, inter, total);
  return fg::check_launch("fg_swiglu");
}

}  // extern "C"
