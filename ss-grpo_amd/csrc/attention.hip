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
//    past the tile only issues its share of the tile loads;
//  * S^T = K Q^T (keys on the M side) puts one query per lane: the online
//    softmax row max / sum are per-lane values plus one exchange with the other
//    half-wave (v_permlane32_swap);
//  * O^T += V^T P^T: P^T is fed straight from the S^T accumulators (bf16) as the
//    B operand; l is summed from the same bf16 P (v_dot2c_f32_bf16);
//  * K/V tiles of 64 keys go from HBM straight into LDS (buffer_load ... lds, the 33
//    1-KB loads of a tile spread over the waves, zeros past the sequence's keys
//    [0, min(seq_len + N, capacity))) through a ring of stages (the layouts and the
//    wait rule are described at the stage constants below); one barrier per tile;
//  * per tile all 16 K fragments are read from LDS before the first MFMA and the
//    16 V fragments (transposed reads) during the S MFMAs (one LDS latency per phase);
//  * the ancestor mask is evaluated only on tiles that reach the tree keys, and
//    the running max (and the O rescale) only moves when a lane's max grows by
//    more than 2^8, so after the first keys the rescale is almost never taken.
// fp32 path: one wave per query row, 64 keys per step, exact online softmax in fp32.
#include "fg_common.h"

#include <algorithm>
#include <type_traits>

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

// LDS stage of one 64-key tile, filled straight from HBM by buffer_load ... lds (each
// 16-byte-per-lane load writes 1 KB of consecutive LDS, lane l at +16 l):
//  * K [64 keys][128 d], rows padded to 17 16-byte chunks (272 B): the S^T MFMA's A
//    fragments (32 keys x 8 d per lane half) are 16-byte reads at compile-time offsets
//    with the 32 rows of a read on distinct banks; the pad chunk loads chunk 15 again;
//  * V [64 keys][128 d] row-major, 16-byte chunk c of key k stored at c ^ 4 (k % 4):
//    the PV A fragments (32 d x 8 keys) are two ds_read_b64_tr_b16 each, whose 16-lane
//    groups then touch all 64 banks once.
constexpr int kKRowB = 272;
constexpr int kKTileB = kKT * kKRowB;        // 17408
constexpr int kVTileB = kKT * kD * 2;        // 16384
constexpr int kStageB = kKTileB + kVTileB;   // 33792
constexpr int kKLoads = kKTileB / 1024;      // 17 1-KB loads
constexpr int kTileLoads = kKLoads + kVTileB / 1024;  // 33
constexpr int stages_for(int w) { return w == 8 ? 4 : 2; }  // 4 x 33 KB with one workgroup per CU
constexpr int loads_per_wave(int w) { return (kTileLoads + w - 1) / w; }

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) v4s lds_v4s;

// s_waitcnt vmcnt(n) leaving the other counters unconstrained (gfx9 encoding).
template <int N>
FG_DEVICE void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <int W>
__global__ void __launch_bounds__(W * 64, 2) tree_attn_bf16_kernel(AttnArgs a, int m_tiles) {
  constexpr int NB = stages_for(W);
  constexpr int LPW = loads_per_wave(W);
  // One array per stage: the compiler tracks the loads into each separately, so
  // reading stage t does not wait for the loads still filling the others.
  __shared__ __attribute__((aligned(1024))) unsigned char st0[kStageB];
  __shared__ __attribute__((aligned(1024))) unsigned char st1[kStageB];
  __shared__ __attribute__((aligned(1024))) unsigned char st2[NB > 2 ? kStageB : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char st3[NB > 3 ? kStageB : 16];
  auto stage = [&](int i) __attribute__((always_inline)) -> unsigned char* {
    return i == 0 ? st0 : i == 1 ? st1 : i == 2 ? st2 : st3;
  };
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

  // ---------------- HBM -> LDS loads: load i of a tile (0..32) is issued by wave i % W.
  // Past the sequence's keys [0, total) the buffer returns 0.
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, total * (kD * 2),
                                                                       0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, total * (kD * 2),
                                                                       0x00020000);
  uint32_t ld_off[LPW];  // byte offset in the tile's global rows of this lane's chunk, per load
#pragma unroll
  for (int u = 0; u < LPW; ++u) {
    const int i = wave + W * u;
    if (i < kKLoads) {
      const int p = i * 64 + lane, row = p / 17, pc = p % 17;
      ld_off[u] = (uint32_t)(row * (kD * 2) + (pc < 16 ? pc : 15) * 16);
    } else {
      const int row = 4 * (i - kKLoads) + (lane >> 4), c = (lane & 15) ^ (4 * (row & 3));
      ld_off[u] = (uint32_t)(row * (kD * 2) + c * 16);
    }
  }
  // Issued as inline asm: the compiler's own tracking of loads into LDS cannot tell
  // the stages apart and would wait for every tile in flight before each LDS read;
  // the waits below (vmcnt before the per-tile barrier) are exact.
  auto load_lds = [&](__amdgpu_buffer_rsrc_t rs, const unsigned char* dst, uint32_t voff)
      __attribute__((always_inline)) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(const lds_void*)dst;
    // s_nop 4: the compiler's hazard checks do not see into inline asm; the load needs a wait
    // state after the M0 write and 5 after any VALU write of the SGPRs it reads.
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(m0) : "memory");
  };
  auto issue_tile = [&](unsigned char* st, int key0) __attribute__((always_inline)) {
    const uint32_t t_off = (uint32_t)key0 * (kD * 2);
#pragma unroll
    for (int u = 0; u < LPW; ++u) {
      const int i = wave + W * u;  // wave-uniform
      if (i < kKLoads)
        load_lds(krs, st + i * 1024, t_off + ld_off[u]);
      else if (i < kTileLoads)
        load_lds(vrs, st + kKTileB + (i - kKLoads) * 1024, t_off + ld_off[u]);
    }
  };
  // this wave's loads per tile (the first waves issue one more)
  const int my_loads = (kTileLoads - wave + W - 1) / W;

  // ---------------- fragment addresses (bytes within a stage)
  const uint32_t k_lane = (uint32_t)(l32 * kKRowB + g * 16);
  // V^T fragment (32 d x 8 keys) via two transposed reads: lane 16 gq + i of a read
  // gets element i % 4 of the 8 bytes addressed by lane 4 j + i / 4 of its group, for
  // j = 0..3. Each lane addresses key 4 (gq / 2) + i / 4 (+ 8 for the second read) and
  // d 32 db + 16 (gq % 2) + 4 (i % 4), so lane l receives keys 4 (l / 32) + j and
  // 8 + 4 (l / 32) + j of d = 32 db + l % 32: the key order of the P^T fragments.
  uint32_t v_lane[kD / 32];
  {
    const int gq = lane >> 4, i = lane & 15, aa = i >> 2;
    const int lowc = 2 * (gq & 1) + ((i & 3) >> 1);
    const uint32_t base = (uint32_t)(kKTileB + (4 * (gq >> 1) + aa) * (kD * 2) + lowc * 16 + 8 * (i & 1));
#pragma unroll
    for (int db = 0; db < kD / 32; ++db) v_lane[db] = base + (uint32_t)(64 * (db ^ aa));
  }

  auto tile_compute = [&](const unsigned char* st, int key0) __attribute__((always_inline)) {
    bf16x8 fr[16];
    // all 16 K fragments before the first MFMA (one LDS latency per tile)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int s = 0; s < kD / 16; ++s)
        fr[kb * 8 + s] = *(const bf16x8*)(st + k_lane + kb * 32 * kKRowB + s * 32);
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
    // the 16 V^T fragments, read during the S MFMAs
#pragma unroll
    for (int db = 0; db < kD / 32; ++db)
#pragma unroll
      for (int ks4 = 0; ks4 < 4; ++ks4) {
        const unsigned char* p0 = st + v_lane[db] + ks4 * 16 * (kD * 2);
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p0);
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p0 + 8 * (kD * 2)));
        fr[db * 4 + ks4] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
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
    // Lazy rescale: the reference max only moves when some lane's max grew by more
    // than 2^kRescaleSlack, so p <= 2^kRescaleSlack and O / l is unchanged.
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
  };

  // ---------------- pipeline: tiles t + 1 .. t + NB - 1 are loading while tile t is
  // computed; one barrier per tile. Loads are issued for NB - 1 tiles past the last
  // (zeros past the sequence's keys) so every wait below has a fixed count.
  const int ntiles = t_end - t_begin;
  const int kbeg = t_begin * kKT;
#pragma unroll
  for (int h = 0; h < NB - 1; ++h) issue_tile(stage(h), kbeg + h * kKT);
  for (int t0 = 0; t0 < ntiles; t0 += NB)
#pragma unroll
  for (int h = 0; h < NB; ++h) {
    if (h > 0 && t0 + h >= ntiles) break;  // uniform over the workgroup
    // this wave's loads of tile t are done once at most NB - 2 tiles of its loads remain
    if (my_loads == LPW)
      wait_vmcnt<(NB - 2) * LPW>();
    else
      wait_vmcnt<(NB - 2) * (LPW - 1)>();
    // Tile t is in LDS for every wave and every wave is done with tile t - 1. No LDS
    // store other than the loads above happens in the loop, so a bare s_barrier after
    // each wave's own vmcnt wait suffices (__syncthreads' release fence would also wait
    // for the loads of the tiles still in flight).
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue_tile(stage((h + NB - 1) % NB), kbeg + (t0 + h + NB - 1) * kKT);
    if (computes) tile_compute(stage(h), kbeg + (t0 + h) * kKT);
  }
  wait_vmcnt<0>();  // no load may still write this workgroup's LDS when it ends

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

// Key-split combine: 8 (sequence, node, q head) rows per 256-thread workgroup, one half-wave
// per row, lane j owning dims 4j .. 4j+3 (16-byte loads of each part's O row).
// O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s (parts with no allowed key have m_s = -inf
// and weigh 0), each sum taken over the parts in order.
constexpr int kCombineRows = 8;

__global__ void __launch_bounds__(256) tree_attn_combine_kernel(AttnArgs a, int rows) {
  const int row = blockIdx.x * kCombineRows + (threadIdx.x >> 5);
  const int lane = threadIdx.x & 31;
  if (row >= rows) return;
  float mx = -INFINITY;
  for (int p = 0; p < a.splits; ++p) mx = fmaxf(mx, a.ml_part[(int64_t)p * rows + row].x);
  float den = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (mx != -INFINITY) {
    for (int p = 0; p < a.splits; ++p) {
      const float2 ml = a.ml_part[(int64_t)p * rows + row];
      if (ml.x == -INFINITY) continue;
      const float w = __builtin_amdgcn_exp2f(ml.x - mx);
      const float4 ov = *(const float4*)(a.o_part + ((int64_t)p * rows + row) * kD + 4 * lane);
      den += w * ml.y;
      o[0] += w * ov.x;
      o[1] += w * ov.y;
      o[2] += w * ov.z;
      o[3] += w * ov.w;
    }
  }
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  *(uint2*)((uint16_t*)a.out + (int64_t)row * kD + 4 * lane) =
      make_uint2(fg::pack_bf16x2(o[0] * inv, o[1] * inv), fg::pack_bf16x2(o[2] * inv, o[3] * inv));
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
    if (split)
      hipLaunchKernelGGL(tree_attn_combine_kernel, dim3((unsigned)((rows + kCombineRows - 1) / kCombineRows)),
                         dim3(256), 0, s, a, (int)rows);
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
