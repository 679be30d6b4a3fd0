// The decoder layer's dense projections (QKV, O, down) as split-K MFMA GEMMs with fp32 partial
// sums, and the kernels that finish them:
//
//   part[s][m, n] = sum over k-steps of split s of x[m, k] * w[n, k]          (fg_linear_parts)
//   x[m] = bf16(x[m] + bf16(sum_s part[s][m])),  h[m] = RMSNorm(x[m]) * g      (fg_residual_rmsnorm_parts)
//
// and, for the QKV projection, the rotary embedding + tree K/V slot write reading the parts
// (fg_rope_kv_write_parts in layers.hip). The residual add rounds the projection to bf16 and then
// the sum, as the Hugging Face decoder layer the reference runs under bf16 autocast does
// (`hidden_states = residual + self.o_proj(...)`, flashgrpo/models/qwen_flashgrpo_wrapper.py:
// 172-180 runs those layers); the parts are summed in split order, so the result does not depend
// on the schedule.
//
// Why split-K: the verify forward's projections have few rows (Qwen2.5-1.5B: 32 sequences x 13
// tree nodes = 416) against long reductions (the down projection: K = 8960), so output tiles alone
// cannot fill 256 CUs; each split takes a contiguous range of k-steps of one output tile.
//
// Tiling (gfx950): one workgroup of 4 waves (2 x 2, one wave's (BM/2) x (BN/2) block each) per
// (output tile, split). K advances 64 per step through an NS-stage LDS ring filled by direct
// HBM->LDS buffer loads (`buffer_load_dwordx4 ... lds`, 1 KB = 8 rows of 128 bytes per instruction),
// 16-byte chunks XOR-swizzled by row so that the fragment reads of 32 consecutive rows hit distinct
// banks. Each k-step is four k16 sub-steps of v_mfma_f32_32x32x16_bf16 with the weight rows as the
// first operand, so each lane ends with 4 consecutive output columns of one row; the fragment reads
// of sub-step s+1 are interleaved with the MFMAs of sub-step s, and the loads of k-step t+NS are
// issued between the MFMAs of k-step t's last sub-step, after the step's one barrier, so NS - 1
// k-steps of loads are in flight while one is computed. At the verify forward's row counts every
// workgroup is resident at once and runs a chain of K / (64 splits) steps, so the time per step
// is the load latency divided by the steps in flight, not the MFMA work: more stages, not more
// workgroups, shorten it.
// Workgroups are numbered so that each XCD takes a contiguous run of tiles along M for one weight
// stripe and split: the stripe is read from HBM once per XCD and reused from its L2.
#include "fg_common.h"

#include <type_traits>


namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kBK = 64;          // K per step
constexpr int kRowBytes = 128;   // one LDS row: kBK bf16
constexpr int kSub = kBK / 16;   // k16 MFMA sub-steps per step

template <int N>
FG_DEVICE void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
FG_DEVICE void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4)); }

// Wait until at most `steps` k-steps of this wave's loads (LPW each) are outstanding, for a
// wave-uniform steps in [0, MAXS] (immediates for s_waitcnt; larger values wait for MAXS).
template <int LPW, int MAXS>
FG_DEVICE void wait_steps(int steps) {
  if constexpr (MAXS >= 3) {
    if (steps >= 3) {
      wait_vmcnt<3 * LPW>();
      return;
    }
  }
  if constexpr (MAXS >= 2) {
    if (steps >= 2) {
      wait_vmcnt<2 * LPW>();
      return;
    }
  }
  if constexpr (MAXS >= 1) {
    if (steps >= 1) {
      wait_vmcnt<LPW>();
      return;
    }
  }
  wait_vmcnt<0>();
}

struct LinArgs {
  const uint16_t* x;  // [rows, ldx]
  int64_t ldx;
  const uint16_t* w;  // [cols, ldw]
  int64_t ldw;
  float* part;        // [splits][rows][cols]
  int64_t part_stride;
  int rows, cols;
  int nks;            // k-steps in total (hidden / 64)
  int ks_per_split;
  int tiles_m, tiles_n, tiles, per_xcd;
  // ROPE epilogue (one split): the QKV projection's bias, rotary embedding and KV-slot write. The
  // weight rows (and bias) of every q and k head are pair-interleaved: row 2j of a head holds its
  // original row j and row 2j + 1 its row j + d/2, so each lane's 4 consecutive output columns
  // are two whole rotary pairs; v heads keep their order.
  const uint16_t* bias;  // [cols] bf16 in the weight's row order, or null
  int num_nodes, q_heads, kv_heads, head_dim;
  const int32_t* seq_len;
  const float2* cos_sin;  // [rows, d/2] (cos, sin) of each row's angles, rounded to bf16
  uint16_t* q_out;  // [rows, q_heads, d]
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t cache_batch, cache_head;
  int capacity;
  const int32_t* row_map;
  int32_t* err_flag;
};

template <int BM, int BN, int NS, bool ROPE = false>
__global__ void __launch_bounds__(256, NS * (BM + BN) * kRowBytes <= 80 * 1024 ? 2 : 1)
    linear_parts_kernel(LinArgs p) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int FM = WM / 32, FN = WN / 32;  // MFMA tiles per wave: rows x columns
  constexpr int A_BYTES = BM * kRowBytes, B_BYTES = BN * kRowBytes, STAGE = A_BYTES + B_BYTES;
  constexpr int LA = BM / 32, LB = BN / 32, LPW = LA + LB;  // 1 KB loads per wave per step
  static_assert(FM >= 1 && FN >= 1 && LA * 4 * 8 == BM && LB * 4 * 8 == BN, "tile sizes: multiples of 64");
  static_assert(NS >= 2 && NS * STAGE <= 160 * 1024 && (NS - 1) * LPW < 64, "ring stages: LDS and vmcnt");
  // ROPE: the epilogue's cos / sin table [BM][BN/2] after the ring is idle
  constexpr int ROPE_LDS = ROPE ? BM * (BN / 2) * 8 : 0;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * STAGE > ROPE_LDS ? NS * STAGE : ROPE_LDS];

  // XCD-aware order: workgroup b runs on XCD b % 8; XCD x takes tiles x*per_xcd .. +per_xcd-1,
  // which walk down M for one (weight stripe, split) before the next.
  const int xcd = blockIdx.x % 8, j = blockIdx.x / 8;
  const int tile = xcd * p.per_xcd + j;
  if (j >= p.per_xcd || tile >= p.tiles) return;  // whole workgroup: before any barrier
  const int tm = tile % p.tiles_m, rest = tile / p.tiles_m;
  const int tn = rest % p.tiles_n, split = rest / p.tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int ks0 = split * p.ks_per_split;
  const int nk = min(p.nks - ks0, p.ks_per_split);  // >= 1: the host makes every split non-empty
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, half = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;

  // ROPE: each lane's rows (one per 32-row MFMA tile) -> cache slot and cache row, and the tile's
  // (row, column pair) entries of the cos / sin table (RE per thread), loaded before the main loop
  // so the loads land while it runs.
  constexpr int RE = ROPE ? BM * (BN / 2) / 256 : 1;
  int r_slot[ROPE ? FM : 1], r_cb[ROPE ? FM : 1];
  float2 t_cs[RE];
  if constexpr (ROPE) {
#pragma unroll
    for (int k = 0; k < FM; ++k) {
      const int m = min(m0 + wm * WM + k * 32 + l32, p.rows - 1);
      const int b = m / p.num_nodes;
      r_slot[k] = p.seq_len[b] + m - b * p.num_nodes;
      r_cb[k] = p.row_map ? p.row_map[b] : b;
    }
    const int hd = p.head_dim / 2;
#pragma unroll
    for (int u = 0; u < RE; ++u) {
      const int e = u * 256 + tid, r = e / (BN / 2), jj = e - r * (BN / 2);
      const int j = ((n0 + 2 * jj) % p.head_dim) / 2;
      t_cs[u] = p.cos_sin[(int64_t)min(m0 + r, p.rows - 1) * hd + j];
    }
  }

  // Buffer descriptors: rows past the matrix end read as zero (rows >= p.rows, columns >= p.cols).
  const int64_t x_bytes = (int64_t)(p.rows - m0) * p.ldx * 2;
  const int64_t w_bytes = (int64_t)(p.cols - n0) * p.ldw * 2;
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x + (int64_t)m0 * p.ldx), (short)0, (int)(x_bytes < 0x7fffffff ? x_bytes : 0x7fffffff), 0x00020000);
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.w + (int64_t)n0 * p.ldw), (short)0, (int)(w_bytes < 0x7fffffff ? w_bytes : 0x7fffffff), 0x00020000);

  // Load lanes: lane l writes LDS bytes l*16 .. of its 1 KB, i.e. row l/8, stored chunk l%8, which
  // holds the row's logical chunk (l%8) ^ (row%8). Wave w loads x rows (w*LA + u)*8 .. and weight
  // rows (w*LB + u)*8 ..
  const int lrow = lane >> 3;
  const int lchunk = (lane & 7) ^ (lrow & 7);
  uint32_t xoff[LA], woff[LB];
#pragma unroll
  for (int u = 0; u < LA; ++u) xoff[u] = (uint32_t)(((wave * LA + u) * 8 + lrow) * p.ldx * 2 + lchunk * 16);
#pragma unroll
  for (int u = 0; u < LB; ++u) woff[u] = (uint32_t)(((wave * LB + u) * 8 + lrow) * p.ldw * 2 + lchunk * 16);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;

  // One 1 KB HBM->LDS load (q < LA: x rows, else weight rows) of k-step ks of this split into ring
  // slot `slot`. M0 holds the LDS address; the s_nop covers the M0-write -> LDS-DMA hazard.
  auto issue = [&](int ks, int slot, int q) __attribute__((always_inline)) {
    const uint32_t koff = (uint32_t)(ks0 + ks) * (kBK * 2);
    const uint32_t sbase = lds0 + slot * STAGE;
    if (q < LA) {
      const uint32_t m0v = sbase + (wave * LA + q) * 1024;
      asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(xoff[q]), "s"(xrs), "s"(koff),
                   "{m0}"(m0v)
                   : "memory");
    } else {
      const uint32_t m0v = sbase + A_BYTES + (wave * LB + q - LA) * 1024;
      asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(woff[q - LA]), "s"(wrs), "s"(koff),
                   "{m0}"(m0v)
                   : "memory");
    }
  };

  // Fragment reads: lane l of a 32-row MFMA tile reads row l%32, k16 sub-step s, 8-element half
  // l/32, i.e. logical chunk 2s + l/32, stored at chunk (2s + l/32) ^ (row % 8).
  uint32_t frag[kSub];
#pragma unroll
  for (int s = 0; s < kSub; ++s) frag[s] = (uint32_t)(l32 * kRowBytes + (((2 * s + half) ^ (l32 & 7)) * 16));
  floatx16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int k = 0; k < FM; ++k)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][k][v] = 0.0f;
  bf16x8 ra[2][FM], rb[2][FN];
  auto read = [&](int slot, int s, int buf) __attribute__((always_inline)) {
    const unsigned char* st = smem + slot * STAGE;
#pragma unroll
    for (int f = 0; f < FM; ++f) ra[buf][f] = *(const bf16x8*)(st + frag[s] + (wm * WM + f * 32) * kRowBytes);
#pragma unroll
    for (int f = 0; f < FN; ++f)
      rb[buf][f] = *(const bf16x8*)(st + A_BYTES + frag[s] + (wn * WN + f * 32) * kRowBytes);
  };
  // One sub-step's MFMAs, the next sub-step's fragment reads placed between them.
  auto mfma_step = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int k = 0; k < FM; ++k)
        acc[i][k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rb[buf][i], ra[buf][k], acc[i][k], 0, 0, 0);
    constexpr int NM = FM * FN, NR = FM + FN, NI = NM < NR ? NM : NR;
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    if constexpr (NM > NI) __builtin_amdgcn_sched_group_barrier(0x008, NM - NI, 0);
    if constexpr (NR > NI) __builtin_amdgcn_sched_group_barrier(0x100, NR - NI, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Prologue: k-steps 0 .. min(NS, nk) - 1 in flight, wait for step 0.
  const int first = min(NS, nk);
#pragma unroll
  for (int h = 0; h < NS; ++h)
    if (h < first) {
#pragma unroll
      for (int q = 0; q < LPW; ++q) issue(h, h, q);
    }
  wait_steps<LPW, NS - 1>(first - 1);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  read(0, 0, 0);

  // k-step t in slot t % NS, which takes k-step t + NS once consumed.
  auto step = [&](int t, auto with_load) __attribute__((always_inline)) {
    const int slot = t % NS;
#pragma unroll
    for (int s = 0; s < kSub - 1; ++s) {
      read(slot, s + 1, (s + 1) & 1);
      mfma_step(s & 1);
    }
    wait_lgkmcnt0();  // this wave's reads of the slot are done
    // k-step t + 1 has landed for this wave; t + 2 .. min(t + NS - 1, nk - 1) may still load
    if constexpr (decltype(with_load)::value)
      wait_vmcnt<(NS - 2) * LPW>();
    else
      wait_steps<LPW, NS - 2>(min(NS - 2, nk - 2 - t));
    __builtin_amdgcn_s_barrier();  // ... and for every wave, and no wave still reads slot t
    __builtin_amdgcn_sched_barrier(0);
    if (t + 1 < nk) read((t + 1) % NS, 0, 0);
    constexpr bool load = decltype(with_load)::value;  // slot t takes k-step t + NS
    constexpr int kLast = (kSub - 1) & 1;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int k = 0; k < FM; ++k) {
        acc[i][k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rb[kLast][i], ra[kLast][k], acc[i][k], 0, 0, 0);
        if constexpr (load) {
          if (i * FM + k < LPW) {
            __builtin_amdgcn_sched_barrier(0);
            issue(t + NS, slot, i * FM + k);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    if constexpr (load) {
#pragma unroll
      for (int q = FM * FN; q < LPW; ++q) issue(t + NS, slot, q);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  int t = 0;
  for (; t + NS < nk; ++t) step(t, std::true_type{});  // NS - 1 steps in flight at each wait
  for (; t < nk; ++t) step(t, std::false_type{});      // the tail: no more loads to issue
  wait_vmcnt<0>();  // no load still writing LDS when the workgroup ends

  // Epilogue: acc[i][k] lane l holds output row m0 + wm*WM + k*32 + l%32 and the columns
  // n0 + wn*WN + i*32 + 8g + 4*(l/32) + 0..3 in elements 4g..4g+3: 16-byte fp32 stores, the two
  // half-waves of a row writing 32 contiguous bytes.
  if constexpr (ROPE) {
    // v = bf16(sum + bias) as the projection's output; q/k pairs (x1, x2) rotated as the rotary
    // kernel rotates them (each product and the sum rounded to bf16, cos / sin rounded to bf16);
    // q rows to q_out, k and v rows to their cache slot (slots outside the cache flag an error).
    const int d = p.head_dim, half_d = d / 2;
    // the tile's cos / sin entries to LDS (the ring is idle after the last step's barrier): lane
    // (row, pair) reads them back after the barrier
    float2* s_cs = (float2*)smem;
#pragma unroll
    for (int u = 0; u < RE; ++u) s_cs[u * 256 + tid] = t_cs[u];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < FM; ++k) {
      const int m = m0 + wm * WM + k * 32 + l32;
      if (m >= p.rows) continue;
      const bool slot_ok = r_slot[k] >= 0 && r_slot[k] < p.capacity;
      if (!slot_ok && p.err_flag) atomicOr(p.err_flag, 8);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * WN + i * 32 + 8 * g + 4 * half;
          if (n >= p.cols) continue;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float bv = p.bias ? fg::bf16_to_f32(p.bias[n + e]) : 0.0f;
            v[e] = fg::round_bf16(acc[i][k][4 * g + e] + bv);
          }
          const int h = n / d, c = n - h * d;
          if (h >= p.q_heads + p.kv_heads) {  // a v head: columns in order
            if (slot_ok)
              *(uint2*)(p.v_cache + (int64_t)r_cb[k] * p.cache_batch +
                        (int64_t)(h - p.q_heads - p.kv_heads) * p.cache_head + (int64_t)r_slot[k] * d + c) =
                  make_uint2(fg::pack_bf16x2(v[0], v[1]), fg::pack_bf16x2(v[2], v[3]));
            continue;
          }
          const int j = c / 2;  // pairs j and j + 1: (v[0], v[1]) and (v[2], v[3])
          float y1[2], y2[2];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const float2 t = s_cs[(wm * WM + k * 32 + l32) * (BN / 2) + (n - n0) / 2 + q];
            const float cs = t.x, sn = t.y;
            const float x1 = v[2 * q], x2 = v[2 * q + 1];
            {
#pragma clang fp contract(off)
              y1[q] = fg::round_bf16(fg::round_bf16(x1 * cs) - fg::round_bf16(x2 * sn));
              y2[q] = fg::round_bf16(fg::round_bf16(x2 * cs) + fg::round_bf16(x1 * sn));
            }
          }
          uint16_t* dst;
          if (h < p.q_heads) {
            dst = p.q_out + ((int64_t)m * p.q_heads + h) * d;
          } else {
            if (!slot_ok) continue;
            dst = p.k_cache + (int64_t)r_cb[k] * p.cache_batch + (int64_t)(h - p.q_heads) * p.cache_head +
                  (int64_t)r_slot[k] * d;
          }
          *(uint32_t*)(dst + j) = fg::pack_bf16x2(y1[0], y1[1]);
          *(uint32_t*)(dst + j + half_d) = fg::pack_bf16x2(y2[0], y2[1]);
        }
    }
    return;
  }
  float* dst = p.part + (int64_t)split * p.part_stride;
#pragma unroll
  for (int k = 0; k < FM; ++k) {
    const int m = m0 + wm * WM + k * 32 + l32;
    if (m >= p.rows) continue;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * WN + i * 32 + 8 * g + 4 * half;
        if (n < p.cols)
          *(float4*)(dst + (int64_t)m * p.cols + n) =
              make_float4(acc[i][k][4 * g], acc[i][k][4 * g + 1], acc[i][k][4 * g + 2], acc[i][k][4 * g + 3]);
      }
  }
}

// table[r][j] = (bf16(cos(pos_r * inv_freq[j])), bf16(sin(pos_r * inv_freq[j]))) for row r = b *
// num_nodes + n at position seq_len[b] + pos_offset[b * pos_stride + n]: the values the rotary
// kernel computes per token, once per forward for every layer's fused epilogue.
__global__ void __launch_bounds__(256) rope_cos_sin_kernel(const int32_t* __restrict__ seq_len,
                                                           const int32_t* __restrict__ pos_offset, int64_t pos_stride,
                                                           const float* __restrict__ inv_freq, int num_nodes, int half,
                                                           int64_t total, float2* __restrict__ table) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= total) return;
  const int64_t r = e / half;
  const int j = (int)(e - r * half);
  const int b = (int)(r / num_nodes), n = (int)(r - (int64_t)b * num_nodes);
  const int pos = seq_len[b] + pos_offset[(int64_t)b * pos_stride + n];
  const float ang = (float)pos * inv_freq[j];
  table[e] = make_float2(fg::round_bf16(cosf(ang)), fg::round_bf16(sinf(ang)));
}

template <int BM, int BN, int NS, bool ROPE>
void launch(LinArgs p, hipStream_t s) {
  p.tiles_m = (p.rows + BM - 1) / BM;
  p.tiles_n = (p.cols + BN - 1) / BN;
  const int splits = (p.nks + p.ks_per_split - 1) / p.ks_per_split;
  p.tiles = p.tiles_m * p.tiles_n * splits;
  p.per_xcd = (p.tiles + 7) / 8;
  hipLaunchKernelGGL((linear_parts_kernel<BM, BN, NS, ROPE>), dim3(8 * p.per_xcd), dim3(256), 0, s, p);
}

template <int BM, int BN, bool ROPE = false>
void launch_stages(LinArgs p, int stages, hipStream_t s) {
  if (stages == 2) launch<BM, BN, 2, ROPE>(p, s);
  else if (stages == 3) launch<BM, BN, 3, ROPE>(p, s);
  else launch<BM, BN, 4, ROPE>(p, s);
}

template <bool ROPE>
void launch_tiles(LinArgs p, int tile_m, int tile_n, int stages, hipStream_t s) {
  if (tile_m == 64 && tile_n == 64)
    launch_stages<64, 64, ROPE>(p, stages, s);
  else if (tile_m == 64)
    launch_stages<64, 128, ROPE>(p, stages, s);
  else if (tile_n == 64)
    launch_stages<128, 64, ROPE>(p, stages, s);
  else
    launch_stages<128, 128, ROPE>(p, stages, s);
}

// x[r] = bf16(x[r] + bf16(sum_s part[s][r])); h[r] = RMSNorm(x[r]) * g. One workgroup per row,
// 8 columns per thread and chunk; the row stays in registers between the two passes.
constexpr int kNormChunks = 4;

__global__ void __launch_bounds__(256) residual_rmsnorm_parts_kernel(const float* __restrict__ part,
                                                                     int64_t part_stride, int splits,
                                                                     uint16_t* __restrict__ x, int64_t ldx,
                                                                     const uint16_t* __restrict__ g,
                                                                     uint16_t* __restrict__ h, int64_t ldh, int H,
                                                                     float eps) {
  const int64_t r = blockIdx.x;
  const int nch = H / 8;
  __shared__ float red[4];
  float v[kNormChunks][8];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int ch = threadIdx.x + c * 256;
    if (ch < nch) {
      const float* src = part + r * H + ch * 8;
      float4 a = *(const float4*)src, b = *(const float4*)(src + 4);
      for (int s = 1; s < splits; ++s) {  // in split order
        const float4 a2 = *(const float4*)(src + s * part_stride), b2 = *(const float4*)(src + s * part_stride + 4);
        a.x += a2.x; a.y += a2.y; a.z += a2.z; a.w += a2.w;
        b.x += b2.x; b.y += b2.y; b.z += b2.z; b.w += b2.w;
      }
      const float y[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      float xv[8];
      fg::load8<fg::kBF16>(x, r * ldx + ch * 8, xv);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[c][e] = fg::round_bf16(xv[e] + fg::round_bf16(y[e]));
      fg::store8<fg::kBF16>(x, r * ldx + ch * 8, v[c]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[c][e] * v[c][e];
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
      fg::load8<fg::kBF16>(g, ch * 8, wv);
      // x * rsqrt(mean x^2 + eps) rounded to bf16, then times the weight (the HF RMSNorm's order)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = wv[e] * fg::round_bf16(v[c][e] * rs);
      fg::store8<fg::kBF16>(h, r * ldh + ch * 8, o);
    }
  }
}

}  // namespace

extern "C" {

int fg_linear_parts(const void* x, int64_t ldx, const void* w, int64_t ldw, float* part, int rows, int cols,
                    int hidden, int splits, int tile_m, int tile_n, int stages, void* stream) {
  FG_REQUIRE(x && w && part, "fg_linear_parts: null pointer");
  FG_REQUIRE(rows > 0 && rows <= (1 << 24) && cols > 0 && cols <= (1 << 24) && hidden > 0,
             "fg_linear_parts: bad shape");
  FG_REQUIRE(hidden % kBK == 0, "fg_linear_parts: hidden size must be a multiple of 64");
  FG_REQUIRE(cols % 4 == 0, "fg_linear_parts: output columns must be a multiple of 4");
  FG_REQUIRE(ldx >= hidden && ldw >= hidden && ldx < (1 << 22) && ldw < (1 << 22), "fg_linear_parts: bad row strides");
  FG_REQUIRE(ldx % 8 == 0 && ldw % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0,
             "fg_linear_parts: x and weight rows must start 16-byte aligned");
  FG_REQUIRE(((uintptr_t)part & 15) == 0, "fg_linear_parts: part must be 16-byte aligned");
  const int nks = hidden / kBK;
  FG_REQUIRE(splits >= 1 && splits <= nks, "fg_linear_parts: splits must be in [1, hidden / 64]");
  const int per = (nks + splits - 1) / splits;
  FG_REQUIRE((nks + per - 1) / per == splits,
             "fg_linear_parts: splits must give every split a k-step (ceil(nk / ceil(nk / splits)) == splits)");
  FG_REQUIRE((tile_m == 64 || tile_m == 128) && (tile_n == 64 || tile_n == 128),
             "fg_linear_parts: tile_m and tile_n must be 64 or 128");
  FG_REQUIRE(stages == 0 || (stages >= 2 && stages <= 4), "fg_linear_parts: stages must be 0 (4), 2, 3 or 4");
  const int64_t tiles = (int64_t)((rows + tile_m - 1) / tile_m) * ((cols + tile_n - 1) / tile_n) * splits;
  FG_REQUIRE(tiles < (1 << 30), "fg_linear_parts: too many tiles");
  LinArgs p{};
  p.x = (const uint16_t*)x;
  p.ldx = ldx;
  p.w = (const uint16_t*)w;
  p.ldw = ldw;
  p.part = part;
  p.part_stride = (int64_t)rows * cols;
  p.rows = rows;
  p.cols = cols;
  p.nks = nks;
  p.ks_per_split = per;
  launch_tiles<false>(p, tile_m, tile_n, stages ? stages : 4, (hipStream_t)stream);
  return fg::check_launch("fg_linear_parts");
}

int fg_rope_cos_sin(const int32_t* seq_len, const int32_t* pos_offset, int64_t pos_batch_stride, const float* inv_freq,
                    int batch, int num_nodes, int head_dim, float* table, void* stream) {
  FG_REQUIRE(seq_len && pos_offset && inv_freq && table, "fg_rope_cos_sin: null pointer");
  FG_REQUIRE(batch > 0 && num_nodes > 0 && head_dim > 0 && head_dim % 2 == 0, "fg_rope_cos_sin: bad shape");
  FG_REQUIRE(pos_batch_stride == 0 || pos_batch_stride >= num_nodes,
             "fg_rope_cos_sin: pos_batch_stride must be 0 or >= num_nodes");
  FG_REQUIRE(((uintptr_t)table & 7) == 0, "fg_rope_cos_sin: table must be 8-byte aligned");
  const int64_t total = (int64_t)batch * num_nodes * (head_dim / 2);
  FG_REQUIRE((total + 255) / 256 < (1ll << 31), "fg_rope_cos_sin: too many rows");
  hipLaunchKernelGGL(rope_cos_sin_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     seq_len, pos_offset, pos_batch_stride, inv_freq, num_nodes, head_dim / 2, total, (float2*)table);
  return fg::check_launch("fg_rope_cos_sin");
}

int fg_linear_rope_kv_write(const void* x, int64_t ldx, const void* w_pairs, int64_t ldw, const void* bias_pairs,
                            int rows, int hidden, int tile_m, int tile_n, int stages, int batch, int num_nodes,
                            int q_heads, int kv_heads, int head_dim, const int32_t* seq_len, const float* cos_sin,
                            void* q_out, void* k_cache, void* v_cache, int64_t cache_batch_stride,
                            int64_t cache_head_stride, int capacity, const int32_t* row_map, int32_t* err_flag,
                            void* stream) {
  FG_REQUIRE(x && w_pairs && seq_len && cos_sin && q_out && k_cache && v_cache,
             "fg_linear_rope_kv_write: null pointer");
  FG_REQUIRE(batch > 0 && num_nodes > 0 && q_heads > 0 && kv_heads > 0 && rows == batch * num_nodes && hidden > 0,
             "fg_linear_rope_kv_write: bad shape (rows must be batch * num_nodes)");
  FG_REQUIRE(head_dim > 0 && head_dim % 8 == 0 && head_dim <= 256,
             "fg_linear_rope_kv_write: head_dim must be a multiple of 8 in [8, 256]");
  FG_REQUIRE(hidden % kBK == 0, "fg_linear_rope_kv_write: hidden size must be a multiple of 64");
  FG_REQUIRE(((uintptr_t)cos_sin & 7) == 0, "fg_linear_rope_kv_write: cos_sin must be 8-byte aligned");
  FG_REQUIRE(ldx >= hidden && ldw >= hidden && ldx < (1 << 22) && ldw < (1 << 22) && ldx % 8 == 0 && ldw % 8 == 0 &&
                 ((uintptr_t)x & 15) == 0 && ((uintptr_t)w_pairs & 15) == 0,
             "fg_linear_rope_kv_write: x and weight rows must start 16-byte aligned");
  FG_REQUIRE((((uintptr_t)q_out | (uintptr_t)k_cache | (uintptr_t)v_cache) & 7) == 0 && cache_batch_stride % 4 == 0 &&
                 cache_head_stride % 4 == 0 && ((uintptr_t)bias_pairs & 7) == 0,
             "fg_linear_rope_kv_write: outputs must be 8-byte aligned");
  FG_REQUIRE((tile_m == 64 || tile_m == 128) && (tile_n == 64 || tile_n == 128),
             "fg_linear_rope_kv_write: tile_m and tile_n must be 64 or 128");
  FG_REQUIRE(stages == 0 || (stages >= 2 && stages <= 4), "fg_linear_rope_kv_write: stages must be 0 (4), 2, 3 or 4");
  const int cols = (q_heads + 2 * kv_heads) * head_dim;
  FG_REQUIRE((int64_t)((rows + tile_m - 1) / tile_m) * ((cols + tile_n - 1) / tile_n) < (1 << 30),
             "fg_linear_rope_kv_write: too many tiles");
  LinArgs p{};
  p.x = (const uint16_t*)x;
  p.ldx = ldx;
  p.w = (const uint16_t*)w_pairs;
  p.ldw = ldw;
  p.rows = rows;
  p.cols = cols;
  p.nks = hidden / kBK;
  p.ks_per_split = p.nks;  // one split: the epilogue holds the whole sum
  p.bias = (const uint16_t*)bias_pairs;
  p.num_nodes = num_nodes;
  p.q_heads = q_heads;
  p.kv_heads = kv_heads;
  p.head_dim = head_dim;
  p.seq_len = seq_len;
  p.cos_sin = (const float2*)cos_sin;
  p.q_out = (uint16_t*)q_out;
  p.k_cache = (uint16_t*)k_cache;
  p.v_cache = (uint16_t*)v_cache;
  p.cache_batch = cache_batch_stride;
  p.cache_head = cache_head_stride;
  p.capacity = capacity;
  p.row_map = row_map;
  p.err_flag = err_flag;
  launch_tiles<true>(p, tile_m, tile_n, stages ? stages : 4, (hipStream_t)stream);
  return fg::check_launch("fg_linear_rope_kv_write");
}

int fg_residual_rmsnorm_parts(const float* part, int splits, int rows, int hidden, void* x, int64_t ldx,
                              const void* weight, float eps, void* h, int64_t ldh, void* stream) {
  FG_REQUIRE(part && x && weight && h, "fg_residual_rmsnorm_parts: null pointer");
  FG_REQUIRE(rows > 0 && splits >= 1 && hidden > 0, "fg_residual_rmsnorm_parts: bad shape");
  FG_REQUIRE(hidden % 8 == 0 && hidden <= 8 * 256 * kNormChunks,
             "fg_residual_rmsnorm_parts: hidden must be a multiple of 8, at most 8192");
  FG_REQUIRE(ldx >= hidden && ldh >= hidden && ldx % 8 == 0 && ldh % 8 == 0,
             "fg_residual_rmsnorm_parts: row strides must be multiples of 8, at least hidden");
  FG_REQUIRE((((uintptr_t)part | (uintptr_t)x | (uintptr_t)weight | (uintptr_t)h) & 15) == 0,
             "fg_residual_rmsnorm_parts: 16-byte alignment");
  hipLaunchKernelGGL(residual_rmsnorm_parts_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, part,
                     (int64_t)rows * hidden, splits, (uint16_t*)x, ldx, (const uint16_t*)weight, (uint16_t*)h, ldh,
                     hidden, eps);
  return fg::check_launch("fg_residual_rmsnorm_parts");
}

}  // extern "C"
