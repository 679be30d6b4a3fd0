// Tree-verify attention over the cached prefix plus the candidate tree.
//
// Query node n of sequence b (all q heads of one KV head, GQA) attends to the
// committed prefix keys [0, seq_len[b]) and to tree keys seq_len[b] + m for
// every node m whose bit is set in the node's 64-bit ancestor-or-self mask
// (with no masks, node n sees new keys 0..n: a causal chain, used by prefill,
// with up to 8192 new keys). The mask is applied to the scores in registers; no
// [B, 1, N, P+N] float mask
// is built (replaces flashgrpo/decoding/tree_attention.py:6-67 feeding the HF
// decoder's eager/SDPA attention, flashgrpo/models/qwen_flashgrpo_wrapper.py:172-180).
//
// bf16 path, one workgroup of W waves per (sequence, kv head, 32W-row query tile),
// W = 8 (one workgroup per CU) when the row tiles fill the chip, else W = 4 (two
// workgroups per CU, more workgroups for the key split):
//  * the query tile is the G*N rows (n-major, G = q heads per kv head) of one
//    KV head, so every K/V tile loaded from HBM serves all of them; the row tiles
//    of one KV head run on one XCD and share its L2;
//  * each wave owns 32 query rows, two waves per SIMD; a wave whose rows are all
//    past the tile only stages K/V;
//  * S^T = K Q^T (keys on the M side) puts one query per lane: the online
//    softmax row max / sum are per-lane values plus one exchange with the other
//    half-wave (v_permlane32_swap);
//  * O^T += V^T P^T: P^T is fed straight from the S^T accumulators (bf16) as the
//    B operand; l is summed from the same bf16 P (v_dot2c_f32_bf16);
//  * the first W/2 waves stage K, the others V, with buffer loads over the
//    sequence's keys [0, min(seq_len + N, capacity)) (loads past the end return 0);
//  * V^T rows hold the 64 keys of a tile in the order 0-3, 8-11, 4-7, 12-15 per
//    16-key block, so the 8 keys a lane feeds the PV MFMA (4g..4g+3 and
//    8+4g..8+4g+3 of a block) are one 16-byte read at a compile-time offset; the
//    staging writes are 4-key runs (8 bytes) with consecutive lanes on consecutive
//    runs of one row, and a row pitch of 9 16-byte chunks puts 8 consecutive rows
//    on distinct banks (reads and writes are conflict-free);
//  * per tile all 16 K fragments are read from LDS before the first MFMA and the
//    16 V^T fragments are read during the S MFMAs (one LDS latency per phase);
//  * K/V tiles are double-buffered in LDS; at the top of iteration t the
//    registers of tile t+1 are stored to the other LDS buffer and the loads of the
//    next tile are issued (W = 8: two register sets, tiles t+2 and t+3 in flight;
//    W = 4: one set, tile t+2); one barrier per 64-key tile;
//  * the ancestor mask is evaluated only on tiles that reach the tree keys, and
//    the running max (and the O rescale) only moves when a lane's max grows by
//    more than 2^8, so after the first keys the rescale is almost never taken.
// fp32 path: one wave per query row, 64 keys per step, exact online softmax in fp32.
#include "fg_common.h"

#include <algorithm>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

struct AttnArgs {
  const void* q;          // [B, N, Hq, d]
  void* out;              // [B, N, Hq, d]
  const void* k;          // layer K cache base [Bc, Hkv, Smax, d]
  const void* v;
  int64_t cache_batch;    // elements
  int64_t cache_head;
  int capacity;           // Smax
  const int32_t* seq_len;
  const int32_t* row_map;
  const uint64_t* anc;    // [anc_batch_stride * B + N] ancestor masks
  int64_t anc_stride;     // 0 when all rows share one topology
  int N, Hq, Hkv, d;
  float scale;
  // Key split: workgroup part `sp` of `splits` covers tiles [sp*tps, (sp+1)*tps) of
  // its row's keys and writes the unnormalised O (fp32) and (max, sum) of each query
  // row to o_part / ml_part ([splits, B, N, Hq, d] and [splits, B, N, Hq]); splits == 1
  // writes the normalised output directly.
  int splits;
  int batch;
  float* o_part;
  float2* ml_part;
};

constexpr int kD = 128;            // head dim of the MFMA path
constexpr int kKT = 64;            // keys per tile
constexpr int kKPitch = kD + 8;    // bf16 elements per K row in LDS
constexpr int kVtPitch = kKT + 8;  // bf16 elements per V^T row in LDS (9 16-byte chunks)
constexpr float kRescaleSlack = 8.0f;  // log2 units
constexpr int rows_tile(int w) { return w * 32; }

FG_DEVICE int c_row32(int i, int lane) { return (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3); }

// Keys key0 .. key0+63 of one row: key0 + j is allowed when it is a prefix key
// (j < sh, sh = seq_len - key0) or tree node j - sh with its bit set in tree_bits.
// Shift amounts are kept in [0, 63].
FG_DEVICE uint64_t tile_allowed_mask(int sh, uint64_t tree_bits) {
  const uint64_t prefix = sh <= 0 ? 0ull : sh >= 64 ? ~0ull : ((1ull << sh) - 1ull);
  const uint64_t tree = sh >= 64 ? 0ull : sh >= 0 ? (tree_bits << sh) : sh <= -64 ? 0ull : (tree_bits >> -sh);
  return prefix | tree;
}
// Bits j < n of a 64-bit mask (n clamped to [0, 64]).
FG_DEVICE uint64_t low_bits(int n) { return n <= 0 ? 0ull : n >= 64 ? ~0ull : ((1ull << n) - 1ull); }

// Position of key k in a V^T row (see the layout notes above).
FG_DEVICE int vt_pos(int k) {
  return (k & ~15) | (k & 3) | (((k >> 3) & 1) << 2) | (((k >> 2) & 1) << 3);
}

// Max / sum of a value with the same lane of the other half-wave.
FG_DEVICE float xor32_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
FG_DEVICE float xor32_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <int W>
__global__ void __launch_bounds__(W * 64, 2) tree_attn_bf16_kernel(AttnArgs a, int m_tiles) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kKT * kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][kD * kVtPitch];
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  constexpr int kRowsTile = rows_tile(W);

  // A unit is one (sequence, kv head, key part); its m_tiles row tiles read the same
  // K/V tiles. Blocks are dispatched round-robin over the 8 XCDs, so the row tiles
  // of a unit are placed 8 blocks apart: one XCD, dispatched together, the second
  // read of each K/V tile served from that XCD's L2.
  int unit = blockIdx.x, mt = 0;
  if (m_tiles > 1) {
    const int grp = blockIdx.x / (8 * m_tiles), rem = blockIdx.x % (8 * m_tiles);
    mt = rem / 8;
    unit = grp * 8 + rem % 8;
    if (unit >= a.batch * a.Hkv * a.splits) return;  // grid padded to whole groups of 8 units
  }
  const int sp = unit % a.splits;
  const int hkv = (unit / a.splits) % a.Hkv;
  const int b = unit / (a.splits * a.Hkv);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int G = a.Hq / a.Hkv;
  const int M = G * a.N;
  const int s0 = a.seq_len[b];
  // Keys past the cache's capacity were never written (fg_rope_kv_write flags them):
  // they are not attended, as in the fp32 kernel.
  const int total = min(s0 + a.N, a.capacity);
  const int nkeys = total;
  const int cb = a.row_map ? a.row_map[b] : b;
  const uint16_t* kbase = (const uint16_t*)a.k + (int64_t)cb * a.cache_batch + (int64_t)hkv * a.cache_head;
  const uint16_t* vbase = (const uint16_t*)a.v + (int64_t)cb * a.cache_batch + (int64_t)hkv * a.cache_head;
  // This workgroup's key tiles [t_begin, t_end) and the key bound they stop at.
  const int tiles_all = (total + kKT - 1) / kKT;
  const int tps = (tiles_all + a.splits - 1) / a.splits;
  const int t_begin = min(sp * tps, tiles_all);
  const int t_end = min(t_begin + tps, tiles_all);
  const int key_end = min(total, t_end * kKT);

  // This lane's query row (column of S^T).
  const int row0 = mt * kRowsTile + wave * 32;
  const bool computes = row0 < M;  // wave-uniform
  const int r = row0 + l32;
  const bool row_ok = r < M;
  const int qn = row_ok ? r / G : 0;
  const int qh = hkv * G + (row_ok ? r % G : 0);
  // anc == NULL: the new keys form a chain (prefill), node qn sees new keys 0..qn
  const uint64_t anc = (row_ok && a.anc) ? a.anc[(int64_t)b * a.anc_stride + qn] : 1ull;
  const uint64_t tree_bits = a.N >= 64 ? anc : anc & ((1ull << a.N) - 1);
  bf16x8 qf[kD / 16];
  {
    const uint16_t* qrow = (const uint16_t*)a.q + (((int64_t)b * a.N + qn) * a.Hq + qh) * kD;
#pragma unroll
    for (int s = 0; s < kD / 16; ++s) {
      uint4 w = row_ok ? *(const uint4*)(qrow + s * 16 + g * 8) : make_uint4(0, 0, 0, 0);
      qf[s] = __builtin_bit_cast(bf16x8, w);
    }
  }
  floatx16 o[kD / 32];
#pragma unroll
  for (int db = 0; db < kD / 32; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const float sl2 = a.scale * 1.44269504088896341f;
  const bf16x2 ones2 = __builtin_bit_cast(bf16x2, 0x3f803f80u);

  // Staging: the first W/2 waves fetch K (thread t: 16-byte chunk t & 15 of keys
  // (t >> 4) + 2W i), the others V (thread t: dims 8 (t >> 4) + 64 u .. +8 of keys
  // 4 (t & 15) + i), both with buffer loads over the sequence's keys [0, nkeys)
  // (past them: 0). CH 16-byte chunks per thread and tile.
  constexpr int CH = 4 * (8 / W);
  constexpr int KROWS = 2 * W;  // K rows between a thread's chunks
  const bool stage_k = __builtin_amdgcn_readfirstlane(wave) < W / 2;  // wave-uniform
  const int st = tid & (W * 32 - 1);
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(stage_k ? kbase : vbase), (short)0, nkeys * (kD * 2), 0x00020000);
  const uint32_t soff = stage_k ? (uint32_t)((st >> 4) * kD + (st & 15) * 8) * 2u
                                : (uint32_t)(4 * (st & 15) * kD + (st >> 4) * 8) * 2u;
  uint16_t* const st_dst = stage_k ? &Ks[0][(st >> 4) * kKPitch + (st & 15) * 8]
                                   : &Vt[0][(8 * (st >> 4)) * kVtPitch + vt_pos(4 * (st & 15))];
  // Byte offset of chunk c from the thread's first chunk.
  auto chunk_off = [&](int c) -> uint32_t {
    return stage_k ? (uint32_t)(c * KROWS * kD * 2) : (uint32_t)((c & 3) * kD * 2 + (c >> 2) * 64 * 2);
  };
  v4u xa[CH], xb[CH];
#define FG_LOAD8(X, KEY0)                                                                         \
  {                                                                                               \
    const uint32_t o_ = soff + (uint32_t)(KEY0) * (uint32_t)(kD * 2);                             \
    _Pragma("unroll") for (int c_ = 0; c_ < CH; ++c_) X[c_] =                                     \
        __builtin_amdgcn_raw_buffer_load_b128(rsrc, o_ + chunk_off(c_), 0, 0);                    \
  }
#define FG_STORE8(X, BUF)                                                                         \
  {                                                                                               \
    if (stage_k) {                                                                                \
      uint16_t* kd_ = st_dst + (BUF) * (kKT * kKPitch);                                           \
      _Pragma("unroll") for (int c_ = 0; c_ < CH; ++c_) *(v4u*)(kd_ + c_ * KROWS * kKPitch) = X[c_]; \
    } else {                                                                                      \
      _Pragma("unroll") for (int u_ = 0; u_ < CH / 4; ++u_) {                                     \
        uint16_t* vd_ = st_dst + (BUF) * (kD * kVtPitch) + u_ * 64 * kVtPitch;                    \
        const v4u* y_ = &X[4 * u_];                                                               \
        _Pragma("unroll") for (int e2 = 0; e2 < 4; ++e2) {                                        \
          *(uint2*)(vd_ + (2 * e2) * kVtPitch) =                                                  \
              make_uint2(__builtin_amdgcn_perm(y_[1][e2], y_[0][e2], 0x05040100u),                \
                         __builtin_amdgcn_perm(y_[3][e2], y_[2][e2], 0x05040100u));               \
          *(uint2*)(vd_ + (2 * e2 + 1) * kVtPitch) =                                              \
              make_uint2(__builtin_amdgcn_perm(y_[1][e2], y_[0][e2], 0x07060302u),                \
                         __builtin_amdgcn_perm(y_[3][e2], y_[2][e2], 0x07060302u));               \
        }                                                                                         \
      }                                                                                           \
    }                                                                                             \
  }

  // Tiles are processed in pairs (LDS buffer 0, then 1); when the count is odd the
  // loop leaves after the first tile of the last pair.
  const int ntiles = t_end - t_begin;
  const int kbeg = t_begin * kKT;
  // Pipeline: while tile t is computed from LDS buffer t % 2, tile t + 1 is already
  // in the other buffer (stored at the top of the iteration, so the store and its
  // wait on the loads overlap the compute). With 8 waves tiles t + 2 and t + 3 are
  // in flight in two register sets; with 4 waves (twice the chunks per thread, two
  // workgroups per CU) tile t + 2 is in flight in one.
  if constexpr (W == 8) {
    FG_LOAD8(xa, kbeg)
    FG_LOAD8(xb, kbeg + kKT)
    FG_STORE8(xa, 0)
    FG_LOAD8(xa, kbeg + 2 * kKT)
  } else {
    FG_LOAD8(xa, kbeg)
    FG_STORE8(xa, 0)
    FG_LOAD8(xa, kbeg + kKT)
  }
  __syncthreads();
  const uint16_t* const kf_src = &Ks[0][l32 * kKPitch + g * 8];
  const uint16_t* const vf_src = &Vt[0][l32 * kVtPitch + g * 8];
  for (int t0 = 0; t0 < ntiles; t0 += 2)
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 1 && t0 + 1 >= ntiles) break;  // uniform over the workgroup
    const int key0 = kbeg + (t0 + h) * kKT;
    if constexpr (W == 8) {
      if (h == 0) {
        FG_STORE8(xb, 1)
        FG_LOAD8(xb, key0 + 3 * kKT)
      } else {
        FG_STORE8(xa, 0)
        FG_LOAD8(xa, key0 + 3 * kKT)
      }
    } else {
      FG_STORE8(xa, h ^ 1)
      FG_LOAD8(xa, key0 + 2 * kKT)
    }

    if (computes) {
      const uint16_t* kf_ = kf_src + h * (kKT * kKPitch);
      const uint16_t* vf_ = vf_src + h * (kD * kVtPitch);
      // All 16 K fragments of the tile are read before the first MFMA (one LDS
      // latency per tile instead of one per fragment pair); the same registers then
      // hold the 16 V^T fragments, read before the exponentials.
      bf16x8 fr[16];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s = 0; s < kD / 16; ++s) fr[kb * 8 + s] = *(const bf16x8*)(kf_ + kb * 32 * kKPitch + s * 16);
      __builtin_amdgcn_sched_barrier(0);
      floatx16 sc[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sc[kb][i] = 0.0f;
#pragma unroll
        for (int s = 0; s < kD / 16; ++s)
          sc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr[kb * 8 + s], qf[s], sc[kb], 0, 0, 0);
      }
#pragma unroll
      for (int db = 0; db < kD / 32; ++db)
#pragma unroll
        for (int c = 0; c < 4; ++c) fr[db * 4 + c] = *(const bf16x8*)(vf_ + db * 32 * kVtPitch + c * 16);
      __builtin_amdgcn_sched_barrier(0);
      if (key0 + kKT > s0 || key0 + kKT > key_end) {  // tile reaches the tree keys or the part's end
        const uint64_t visible = a.anc ? tile_allowed_mask(s0 - key0, tree_bits) : low_bits(s0 + qn + 1 - key0);
        const uint64_t allowed = (visible & low_bits(key_end - key0)) >> (g * 4);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const bool ok = (allowed >> (kb * 32 + c_row32(i, 0))) & 1ull;
            sc[kb][i] = ok ? sc[kb][i] : -INFINITY;
          }
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, sc[kb][i]);
      const float m_new = fmaxf(m_run, xor32_max(tmax) * sl2);
      // Lazy rescale: the reference max only moves when some lane's max grew by
      // more than 2^kRescaleSlack, so p <= 2^kRescaleSlack and O / l is unchanged.
      if (__any(m_new > m_run + kRescaleSlack)) {
        const float m_sub = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_sub);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < kD / 32; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
        m_run = m_new;
      }
      const float m_sub = m_run == -INFINITY ? 0.0f : m_run;
      float psum = l_run;
      bf16x8 pf[2][2];  // [kb][ks] B operand of P^T
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          uint32_t packed[4];
#pragma unroll
          for (int j = 0; j < 8; j += 2) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[kb][ks * 8 + j], sl2, -m_sub));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[kb][ks * 8 + j + 1], sl2, -m_sub));
            packed[j / 2] = fg::pack_bf16x2(p0, p1);
            psum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, packed[j / 2]), ones2, psum, false);
          }
          pf[kb][ks] = __builtin_bit_cast(bf16x8, make_uint4(packed[0], packed[1], packed[2], packed[3]));
        }
      l_run = psum;
#pragma unroll
      for (int db = 0; db < kD / 32; ++db)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
            o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr[db * 4 + kb * 2 + ks], pf[kb][ks], o[db], 0, 0, 0);
    }
    __syncthreads();
  }
#undef FG_LOAD8
#undef FG_STORE8

  const float l = xor32_sum(l_run);
  if (a.splits > 1) {  // unnormalised part: O rows (fp32) and (max in log2 units, sum)
    if (row_ok) {
      const int64_t prow = (((int64_t)sp * a.batch + b) * a.N + qn) * a.Hq + qh;
      float* orow = a.o_part + prow * kD;
#pragma unroll
      for (int db = 0; db < kD / 32; ++db)
#pragma unroll
        for (int i = 0; i < 16; i += 4)
          *(float4*)(orow + db * 32 + c_row32(i, lane)) = make_float4(o[db][i], o[db][i + 1], o[db][i + 2], o[db][i + 3]);
      if (g == 0) a.ml_part[prow] = make_float2(m_run, l);
    }
    return;
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  if (row_ok) {
    uint16_t* orow = (uint16_t*)a.out + (((int64_t)b * a.N + qn) * a.Hq + qh) * kD;
#pragma unroll
    for (int db = 0; db < kD / 32; ++db)
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        const int d0 = db * 32 + c_row32(i, lane);
        const uint32_t w0 = fg::pack_bf16x2(o[db][i] * inv, o[db][i + 1] * inv);
        const uint32_t w1 = fg::pack_bf16x2(o[db][i + 2] * inv, o[db][i + 3] * inv);
        *(uint2*)(orow + d0) = make_uint2(w0, w1);
      }
  }
}

// Key-split combine: one wave per (sequence, node, q head) row; lane j owns dims
// 2j, 2j+1. O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s (parts with no
// allowed key have m_s = -inf and weigh 0).
__global__ void __launch_bounds__(64) tree_attn_combine_kernel(AttnArgs a, int rows) {
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  float mx = -INFINITY;
  for (int p = 0; p < a.splits; ++p) mx = fmaxf(mx, a.ml_part[(int64_t)p * rows + row].x);
  float den = 0.0f, o0 = 0.0f, o1 = 0.0f;
  if (mx != -INFINITY) {
    for (int p = 0; p < a.splits; ++p) {
      const float2 ml = a.ml_part[(int64_t)p * rows + row];
      if (ml.x == -INFINITY) continue;
      const float w = __builtin_amdgcn_exp2f(ml.x - mx);
      const float2 ov = *(const float2*)(a.o_part + ((int64_t)p * rows + row) * kD + 2 * lane);
      den += w * ml.y;
      o0 += w * ov.x;
      o1 += w * ov.y;
    }
  }
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  *(uint32_t*)((uint16_t*)a.out + (int64_t)row * kD + 2 * lane) = fg::pack_bf16x2(o0 * inv, o1 * inv);
}

// fp32: one wave per (sequence, node, q head), 64 keys per step. Lane j scores key
// key0 + j (dot product over the head dim from float4 loads against q in LDS); the
// step's max and sum are wave reductions; PV broadcasts each key's p with v_readlane
// while lane j accumulates dims j and j + 64 of O (exact online softmax, fp32). All
// loads of a step are independent and unconditional (addresses clamped to the last
// key), so each step waits for memory about once per phase.
template <int D>
__global__ void __launch_bounds__(64) tree_attn_f32_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float qs[D];
  const int qh = blockIdx.x % a.Hq;
  const int n = (blockIdx.x / a.Hq) % a.N;
  const int b = blockIdx.x / (a.Hq * a.N);
  const int lane = threadIdx.x;
  const int G = a.Hq / a.Hkv, hkv = qh / G;
  const int s0 = a.seq_len[b];
  const int cb = a.row_map ? a.row_map[b] : b;
  const float* kbase = (const float*)a.k + (int64_t)cb * a.cache_batch + (int64_t)hkv * a.cache_head;
  const float* vbase = (const float*)a.v + (int64_t)cb * a.cache_batch + (int64_t)hkv * a.cache_head;
  const float* qrow = (const float*)a.q + (((int64_t)b * a.N + n) * a.Hq + qh) * D;
  const uint64_t anc = a.anc ? a.anc[(int64_t)b * a.anc_stride + n] : 0ull;
  for (int j = lane; j < D; j += 64) qs[j] = qrow[j];
  __syncthreads();
  float m = -INFINITY, l = 0.0f, o0 = 0.0f, o1 = 0.0f;
  const int total = min(s0 + a.N, a.capacity);
  for (int key0 = 0; key0 < total; key0 += 64) {
    const int key = key0 + lane;
    const bool ok = key < total && (key < s0 || (a.anc ? ((anc >> (key - s0)) & 1ull) != 0 : key <= s0 + n));
    const float* kr = kbase + (int64_t)min(key, total - 1) * D;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < D; j += 4) {
      const float4 kv = *(const float4*)(kr + j);
      const float4 qv = *(const float4*)(qs + j);
      acc = fmaf(qv.x, kv.x, acc);
      acc = fmaf(qv.y, kv.y, acc);
      acc = fmaf(qv.z, kv.z, acc);
      acc = fmaf(qv.w, kv.w, acc);
    }
    const float s = ok ? acc * a.scale : -INFINITY;
    const float m_new = fmaxf(m, fg::wave_max(s));
    if (m_new == -INFINITY) continue;  // wave-uniform: no allowed key yet
    const float alpha = expf(m - m_new);
    const float p = ok ? expf(s - m_new) : 0.0f;
    l = l * alpha + fg::wave_sum(p);
    o0 *= alpha;
    o1 *= alpha;
    // Keys past the end carry p = 0 and read the last key's row, so they add 0.
    const int last = total - 1 - key0;
    const float* vr = vbase + (int64_t)key0 * D + lane;
#pragma unroll
    for (int j = 0; j < 64; ++j) {
      const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), j));
      const float* v_ = vr + (int64_t)min(j, last) * D;
      if (D > 0) o0 = fmaf(pj, lane < D ? v_[0] : 0.0f, o0);
      if (D > 64) o1 = fmaf(pj, v_[64], o1);
    }
    m = m_new;
  }
  float* orow = (float*)a.out + (((int64_t)b * a.N + n) * a.Hq + qh) * D;
  if (lane < D) orow[lane] = o0 / l;
  if (lane + 64 < D) orow[lane + 64] = o1 / l;
}


// Waves per workgroup of the bf16 kernel: 8 (one workgroup per CU, every K/V tile
// staged once per CU) when the row tiles fill the 256 CUs; otherwise 4 (two
// workgroups per CU, twice as many workgroups for the key split). Measured at the
// 7B tree shape: 64 sequences 85 us with 8 waves vs 96 with 4; 4 sequences 28 vs 23.5.
int attn_waves(int batch, int num_nodes, int q_heads, int kv_heads) {
  const int M = (q_heads / kv_heads) * num_nodes;
  return batch * kv_heads * ((M + rows_tile(8) - 1) / rows_tile(8)) >= 256 ? 8 : 4;
}

// Key-split policy: when (sequences x kv heads x row tiles) leaves workgroup slots
// idle, each workgroup's keys are cut into parts of at least 8 tiles (capacity
// bound); shorter parts measured no faster than one workgroup per row tile.
constexpr int kMaxSplits = 16;

int attn_splits(int batch, int num_nodes, int q_heads, int kv_heads, int capacity) {
  const int w = attn_waves(batch, num_nodes, q_heads, kv_heads);
  const int target = 256 * (8 / w);  // workgroups that fill the chip
  const int M = (q_heads / kv_heads) * num_nodes;
  const int base = batch * kv_heads * ((M + rows_tile(w) - 1) / rows_tile(w));
  if (base >= target) return 1;
  const int tiles = (capacity + kKT - 1) / kKT;
  const int sp = std::min((target + base - 1) / base, std::max(1, tiles / 8));
  return std::max(1, std::min(sp, kMaxSplits));
}

size_t attn_workspace_bytes(int splits, int batch, int num_nodes, int q_heads) {
  if (splits <= 1) return 0;
  const size_t rows = (size_t)splits * batch * num_nodes * q_heads;
  return rows * (kD * sizeof(float) + sizeof(float2)) + 256;
}

template <int W>
void launch_attn_bf16(const AttnArgs& a, int M, hipStream_t s) {
  const int m_tiles = (M + rows_tile(W) - 1) / rows_tile(W);
  const int units = a.batch * a.Hkv * a.splits;
  const int blocks = m_tiles > 1 ? (units + 7) / 8 * 8 * m_tiles : units;
  hipLaunchKernelGGL(tree_attn_bf16_kernel<W>, dim3(blocks), dim3(W * 64), 0, s, a, m_tiles);
}

}  // namespace

extern "C" size_t fg_tree_attention_workspace(int batch, int num_nodes, int q_heads, int kv_heads, int head_dim,
                                              int capacity) {
  if (batch <= 0 || num_nodes <= 0 || q_heads <= 0 || kv_heads <= 0 || head_dim != kD || capacity <= 0) return 0;
  return attn_workspace_bytes(attn_splits(batch, num_nodes, q_heads, kv_heads, capacity), batch, num_nodes,
                              q_heads);
}

extern "C" int fg_tree_attention(const void* q, void* out, const void* k_cache, const void* v_cache, int dtype,
                                 int batch, int num_nodes, int q_heads, int kv_heads, int head_dim,
                                 int64_t cache_batch_stride, int64_t cache_head_stride, int capacity,
                                 const int32_t* seq_len, const int32_t* row_map, const uint64_t* anc,
                                 int64_t anc_batch_stride, float scale, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  FG_REQUIRE(q && out && k_cache && v_cache && seq_len, "fg_tree_attention: null pointer");
  FG_REQUIRE(batch > 0 && num_nodes > 0 && (anc ? num_nodes <= 64 : num_nodes <= 8192),
             "fg_tree_attention: num_nodes must be in [1, 64] with masks, [1, 8192] for a chain");
  FG_REQUIRE(q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0, "fg_tree_attention: heads");
  FG_REQUIRE(capacity >= num_nodes, "fg_tree_attention: capacity");
  AttnArgs a;
  a.q = q; a.out = out; a.k = k_cache; a.v = v_cache;
  a.cache_batch = cache_batch_stride; a.cache_head = cache_head_stride; a.capacity = capacity;
  a.seq_len = seq_len; a.row_map = row_map; a.anc = anc; a.anc_stride = anc_batch_stride;
  a.N = num_nodes; a.Hq = q_heads; a.Hkv = kv_heads; a.d = head_dim; a.scale = scale;
  a.splits = 1; a.batch = batch; a.o_part = nullptr; a.ml_part = nullptr;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == fg::kBF16) {
    FG_REQUIRE(head_dim == kD, "fg_tree_attention: bf16 path supports head_dim 128");
    FG_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)k_cache & 15) == 0 && ((uintptr_t)v_cache & 15) == 0 &&
                   cache_head_stride % 8 == 0 && cache_batch_stride % 8 == 0,
               "fg_tree_attention: 16-byte alignment");
    FG_REQUIRE((int64_t)capacity * kD * 2 < (1ll << 31), "fg_tree_attention: capacity too large");
    const int M = (q_heads / kv_heads) * num_nodes;
    const int splits = attn_splits(batch, num_nodes, q_heads, kv_heads, capacity);
    const bool split = splits > 1 && workspace &&
                       workspace_bytes >= attn_workspace_bytes(splits, batch, num_nodes, q_heads);
    const size_t rows = (size_t)batch * num_nodes * q_heads;
    if (split) {
      char* w = (char*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
      a.splits = splits;
      a.o_part = (float*)w;
      a.ml_part = (float2*)(w + (size_t)splits * rows * kD * sizeof(float));
    }
    if (attn_waves(batch, num_nodes, q_heads, kv_heads) == 8)
      launch_attn_bf16<8>(a, M, s);
    else
      launch_attn_bf16<4>(a, M, s);
    if (split) hipLaunchKernelGGL(tree_attn_combine_kernel, dim3((unsigned)rows), dim3(64), 0, s, a, (int)rows);
  } else if (dtype == fg::kF32) {
    FG_REQUIRE(head_dim == 64 || head_dim == 128, "fg_tree_attention: fp32 path supports head_dim 64 or 128");
    FG_REQUIRE(((uintptr_t)k_cache & 15) == 0 && cache_head_stride % 4 == 0 && cache_batch_stride % 4 == 0,
               "fg_tree_attention: fp32 path needs 16-byte aligned K rows");
    if (head_dim == 64)
      hipLaunchKernelGGL(tree_attn_f32_kernel<64>, dim3(batch * num_nodes * q_heads), dim3(64), 0, s, a);
    else
      hipLaunchKernelGGL(tree_attn_f32_kernel<128>, dim3(batch * num_nodes * q_heads), dim3(64), 0, s, a);
  } else {
    return fg::fail("fg_tree_attention: dtype");
  }
  return fg::check_launch("fg_tree_attention");
}
