// Tied LM head over up to 256 rows with the weight streamed once, and the per-row
// top-k candidates and (max, sum of exp) of the logits produced in the epilogue.
//
//   logits[m, n] = x[rows ? rows[m] : m, :] . w[n, :]        m < M <= 256, n < N
//
// Replaces the lm_head projections of flashgrpo/decoding/flash_medusa_decoder.py:289-294
// (Medusa rows), :1079-1091 (leaf / next-round rows) and the per-depth torch.topk of
// flashgrpo/decoding/medusa_tree.py:239-252 that reads those logits back.
//
// Work split: the vocabulary is cut into 32-column blocks dealt out in contiguous runs to
// every wave of a persistent grid (one workgroup of 8 waves per CU). A wave streams its
// block's 32 weight rows from HBM into registers as whole 128-byte row pieces (8 lanes per
// row, 4 loads per 64-wide k-step; this measured 0.76 of HBM against 0.65 for loading the
// MFMA operand layout directly), turns them into the operand layout through its own 4 KB
// of LDS, and multiplies them with v_mfma_f32_32x32x16_bf16 against the activation rows,
// which the workgroup stages per k-step in LDS (HBM -> LDS loads, 3-4 stages). 16-byte
// pieces are XOR-swizzled in both LDS layouts. MFMA step kk of a k-step uses 16-byte piece
// 4 g + kk of each row for lane group g, on both operands, so both sum the same products.
// The weight is read exactly once; the activations (<= 1.8 MB) are re-read from L2 per
// block round.
//
// Epilogue of a block round: the logits are written (optional); without top-k, each row's
// maximum and first maximum over the workgroup's columns can be kept (part_max / part_key,
// one part per workgroup: the row maxima a sampler needs before it can weigh the logits);
// with top-k the
// workgroup's 256 columns x M rows are rounded to bf16 (the values the reference ranks)
// and placed in LDS, where each row's running top-K and (max, sum exp) over the
// workgroup's columns are updated. At the end every workgroup writes its part of each
// row to part_keys / part_lse, which topk_phase2 (topk.hip) merges per row.
#include "fg_common.h"
#include "fg_topk.h"

#include <algorithm>
#include <mutex>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kBlocks = 8;  // 32-column blocks per workgroup and round (W waves x NB blocks)
constexpr int kKS = 64;     // k-step
constexpr int kTileRow = 528;  // bytes per row of the epilogue's bf16 tile (256 columns + 16)
// k-steps in flight; the activation ring has one stage more
constexpr int dist_for(int mi) { return mi >= 8 ? 2 : 3; }
// Waves per workgroup (W waves x NB = 8 / W blocks of 32 columns). A layout of 4 waves x 2
// blocks at 256 rows (one wave per SIMD, the accumulators in 256 AGPRs) would read each
// activation fragment once for two blocks, halving the LDS reads that bound the 8-wave
// layout there; built, it returned wrong logits for the row blocks whose accumulators sit in
// AGPRs 0-63 and 128-191 (the compiler moves accumulators between AGPRs and VGPRs around the
// asm-issued weight loads), so every row count runs 8 waves.
constexpr int waves_for(int) { return 8; }

template <int N>
FG_DEVICE void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// 16-byte piece position of piece c of activation row r in LDS (rows of 128 bytes). The
// swizzle depends on r % 32 only, so every 32-row block has the same layout.
FG_DEVICE int a_swz(int r) { return (r ^ ((r >> 3) & 3)) & 7; }
FG_DEVICE int a_pos(int r, int c) { return c ^ a_swz(r); }

struct LmArgs {
  const void* x;
  int64_t ldx;
  const int32_t* rows;        // optional row gather
  const int32_t* row_active;  // optional: nothing is computed when every flag is 0
  int M, K;
  const void* w;
  int64_t ldw;
  int N;
  void* out;  // optional [M, ldo]
  int64_t ldo;
  uint64_t* part_keys;  // [M, nparts, KT]
  float2* part_lse;     // [M, nparts]
  float* part_max;      // [M, nparts] (PM): max of the stored logits, NaN ignored
  uint64_t* part_key;   // [M, nparts] (PM): largest rank key (the first maximum, NaN first)
  int nparts;  // = grid: one part per workgroup
  // Medusa fc (MED): `heads` products of the same shape, x, w and out advancing per head,
  // each cut into `ksplit` key ranges. Workgroup task t = (h * ksplit + p) * ngroups + c
  // computes columns [256 c, 256 c + 256) of head h over k-steps
  // [p * KST / ksplit, (p + 1) * KST / ksplit) into fp32 rows (p * heads + h) * M + m of out.
  int heads, ksplit, ngroups;
  int64_t x_head_bytes, w_head_bytes;
};

template <int MI, int CDT, int KT, bool SAN, bool PM, int W, bool MED = false>
__global__ void __launch_bounds__(W * 64, 1) lm_stream_kernel(LmArgs a) {
  static_assert(!PM || KT == 0, "row maxima parts come with the logits-only epilogue");
  static_assert(!MED || (KT == 0 && !PM && CDT == fg::kF32), "Medusa tasks write fp32 partial sums only");
  constexpr int NB = kBlocks / W;  // 32-column blocks per wave and round
  static_assert(NB * W == kBlocks, "waves");
  constexpr int kDist = dist_for(MI), kStages = kDist + 1;
  constexpr int MP = MI * 32;
  constexpr int STAGE = MP * 128;
  constexpr int LA = STAGE / 1024 / W;  // HBM -> LDS loads per wave and k-step
  constexpr int LB = 4 * NB;            // weight loads per lane and k-step
  constexpr int L = LA + LB;
  static_assert(MI % 2 == 0 && LA >= 1, "rows");
  static_assert((kDist - 1) * L < 64, "vmcnt");
  constexpr int XPOSE = kStages * STAGE;     // per-wave NB x 4 KB weight transpose buffers
  constexpr int TILE = KT ? MP * kTileRow : 0;
  constexpr int MAIN = XPOSE + kBlocks * 4096 > TILE ? XPOSE + kBlocks * 4096 : TILE;
  // each row's running top-KT keys and (max, sum exp) over this workgroup's columns
  constexpr int LISTS = KT ? MP * (KT * 8 + 8) : 0;
  constexpr int LDS = MAIN + LISTS;
  static_assert(LDS <= 160 * 1024 - 256, "LDS");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[LDS];
  uint64_t* s_keys = (uint64_t*)(smem + MAIN);
  float2* s_lse = (float2*)(smem + MAIN + MP * KT * 8);
  __shared__ int s_n0[kBlocks], s_nv[kBlocks], s_any;

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (a.row_active) {
    if (tid == 0) s_any = 0;
    __syncthreads();
    if (tid < a.M && a.row_active[tid]) s_any = 1;
    __syncthreads();
    if (!s_any) return;
  }
  // Wave block (NB x 32 columns) rd * GW + gw goes to wave gw = wave * G + workgroup in round
  // rd: the blocks of a partial last round are spread over every CU (a CU's loads, not HBM,
  // bound a round that only a few CUs run).
  const int nblk = (a.N + 32 * NB - 1) / (32 * NB);
  const int gw_total = gridDim.x * W;
  const int gw = wave * gridDim.x + blockIdx.x;
  const int q = nblk / gw_total, rem = nblk % gw_total;
  const int my_cnt = q + (gw < rem ? 1 : 0);
  // wave 0 has the most blocks; Medusa tasks are dealt out per workgroup (grid <= tasks)
  const int rounds = MED ? (a.heads * a.ksplit * a.ngroups - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x
                         : q + ((int)blockIdx.x < rem ? 1 : 0);
  const int KST = a.K / kKS;

  // activation staging: load u of this wave fills LDS rows (wave * LA + u) * 8 + lane / 8
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, -1, 0x00020000);
  uint32_t xoff[LA];
#pragma unroll
  for (int u = 0; u < LA; ++u) {
    const int r = (wave * LA + u) * 8 + (lane >> 3);
    const int m = min(r, a.M - 1);
    const int src = a.rows ? a.rows[m] : m;
    xoff[u] = (uint32_t)((int64_t)src * a.ldx * 2) + (uint32_t)(a_pos(r, lane & 7) * 16);
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem + wave * LA * 1024;
  // koff: byte offset of the k-step within the rows (plus the head's offset for MED)
  auto issue_x = [&](uint32_t koff, int stage) __attribute__((always_inline)) {
    const uint32_t st = (uint32_t)stage * STAGE;
#pragma unroll
    for (int u = 0; u < LA; ++u) {
      const uint32_t m0v = lds0 + st + u * 1024;
      // s_nop 4: the compiler's hazard checks do not see into inline asm, so the asm keeps
      // the wait states a load needs after a VALU write of an SGPR it reads (5; the compiler
      // moves spilled SGPRs back with v_readlane) and after the M0 write (1).
      asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(xoff[u]), "s"(xrs), "s"(koff),
                   "{m0}"(m0v)
                   : "memory");
    }
  };
  // weight stream: load q of a k-step brings rows q * 8 + lane / 8 of the wave block,
  // 16-byte piece lane % 8 (128 contiguous bytes per row)
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, -1, 0x00020000);
  uint32_t woff[LB];
  v4u wr[kDist][LB];
  // Issued as inline asm so the compiler adds no waits of its own: it would count only these
  // loads, not the activation loads between them, and wait for younger k-steps too. The
  // static wait before each k-step's barrier covers them.
  // (one statement with its own wait states, as for the activation loads)
  auto issue_w = [&](v4u(&dst)[LB], int koff) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < NB; ++h)
      asm volatile(
          "s_nop 4\n\t"
          "buffer_load_dwordx4 %0, %4, %8, %9 offen\n\t"
          "buffer_load_dwordx4 %1, %5, %8, %9 offen\n\t"
          "buffer_load_dwordx4 %2, %6, %8, %9 offen\n\t"
          "buffer_load_dwordx4 %3, %7, %8, %9 offen"
          : "=&v"(dst[4 * h]), "=&v"(dst[4 * h + 1]), "=&v"(dst[4 * h + 2]), "=&v"(dst[4 * h + 3])
          : "v"(woff[4 * h]), "v"(woff[4 * h + 1]), "v"(woff[4 * h + 2]), "v"(woff[4 * h + 3]), "s"(wrs),
            "s"(koff));
  };
  // this wave's transpose buffer: row r of the wave block at r * 128 (block nb at nb * 4 KB),
  // pieces swizzled like x
  unsigned char* xp = smem + XPOSE + wave * 4096 * NB;
  uint32_t xw[LB];
#pragma unroll
  for (int q = 0; q < LB; ++q) {
    const int r = q * 8 + (lane >> 3);
    xw[q] = (uint32_t)(r * 128 + a_pos(r, lane & 7) * 16);
  }
  // A fragment address of m-block 0, piece kk of this lane's group (bytes within a stage)
  uint32_t foff[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) foff[kk] = (uint32_t)(l32 * 128 + a_pos(l32, g * 4 + kk) * 16);
  // PM: running maximum and best rank key of row 32 i + l32 over this lane's columns
  float pm_max[PM ? MI : 1];
  uint64_t pm_key[PM ? MI : 1];
#pragma unroll
  for (int i = 0; i < (PM ? MI : 1); ++i) {
    pm_max[i] = -INFINITY;
    pm_key[i] = 0;
  }

  for (int rd = 0; rd < rounds; ++rd) {
    // Every wave issues the same loads every k-step, so the waits below are static: a wave
    // without a block this round, and the k-steps past the last, re-read one cached line.
    bool active = rd < my_cnt;  // wave-uniform
    int n0 = (rd * gw_total + gw) * 32 * NB;
    // k-steps [kb, kb + kst) (workgroup-uniform); xb / wb: byte offsets of the first k-step
    // in x and in this wave's weight rows; orow: first output row
    int kb = 0, kst = KST;
    uint32_t xb = 0, wb = 0;
    int64_t orow = 0;
    if constexpr (MED) {
      const int t = rd * (int)gridDim.x + (int)blockIdx.x;
      const int c = t % a.ngroups, hp = t / a.ngroups, p = hp % a.ksplit, h = hp / a.ksplit;
      n0 = c * (32 * kBlocks) + wave * 32 * NB;
      active = n0 < a.N;
      kb = p * KST / a.ksplit;
      kst = (p + 1) * KST / a.ksplit - kb;
      xb = (uint32_t)(h * a.x_head_bytes) + (uint32_t)kb * (kKS * 2);
      wb = active ? (uint32_t)(h * a.w_head_bytes) + (uint32_t)kb * (kKS * 2) : 0u;
      orow = (int64_t)(p * a.heads + h) * a.M;
    }
#pragma unroll
    for (int q = 0; q < LB; ++q)
      woff[q] = active ? (uint32_t)((int64_t)min(n0 + q * 8 + (lane >> 3), a.N - 1) * a.ldw * 2) +
                             (uint32_t)((lane & 7) * 16)
                       : 0u;
    const int wstep = active ? kKS * 2 : 0;
    const uint32_t xstep = kKS * 2;
    floatx16 acc[MI][NB];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][nb][v] = 0.0f;

#pragma unroll
    for (int h = 0; h < kDist; ++h) {
      issue_x(xb + (h < kst ? h : 0) * xstep, h % kStages);
      issue_w(wr[h], wb + (h < kst ? h * wstep : 0));
    }
    for (int k0 = 0; k0 < kst; k0 += kDist) {
#pragma unroll
      for (int sl = 0; sl < kDist; ++sl) {
        const int ks = k0 + sl;
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<(kDist - 1) * L>();  // k-step ks has landed (younger ones may be in flight)
        // k-step ks is in LDS for every wave, and every wave is done with ks - 1
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const int kn = ks + kDist;
        issue_x(xb + (kn < kst ? kn : 0) * xstep, kn % kStages);
        if (ks < kst && active) {
          const unsigned char* st = smem + (ks % kStages) * STAGE;
          // the weight pieces into operand layout (this wave read the previous ones already)
#pragma unroll
          for (int q = 0; q < LB; ++q) *(v4u*)(xp + xw[q]) = wr[sl][q];
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            bf16x8 bf[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) bf[nb] = *(const bf16x8*)(xp + nb * 4096 + foff[kk]);
#pragma unroll
            for (int i = 0; i < MI; ++i) {
              const bf16x8 af = *(const bf16x8*)(st + i * 32 * 128 + foff[kk]);
#pragma unroll
              for (int nb = 0; nb < NB; ++nb)
                acc[i][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[nb], af, acc[i][nb], 0, 0, 0);
            }
            // one piece's fragments live at a time (hoisting all four would spill at 256 rows)
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        // the weight slot is free once its pieces are in LDS
        issue_w(wr[sl], wb + (kn < kst ? kn * wstep : 0));
      }
    }
    wait_vmcnt<0>();
    // The last k-steps' weight loads are never read: keep their registers allocated until
    // they have landed, or the compiler could give them to the code below while the loads
    // still write them.
#pragma unroll
    for (int h = 0; h < kDist; ++h)
#pragma unroll
      for (int q4 = 0; q4 < LB; q4 += 4)
        asm volatile("" ::"v"(wr[h][q4]), "v"(wr[h][q4 + 1]), "v"(wr[h][q4 + 2]), "v"(wr[h][q4 + 3]));
    __builtin_amdgcn_sched_barrier(0);

    // acc[i][nb] is a tile of C^T: lane holds row m = 32 i + l32, columns
    // n0 + 32 nb + 8 (v / 4) + 4 g + v % 4
    if (a.out && active) {
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = i * 32 + l32;
        if (m >= a.M || (a.row_active && !a.row_active[m])) continue;  // inactive rows stay unwritten
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          const int n = n0 + nb * 32 + v4 * 8 + g * 4;
          if (n >= a.N) continue;
          if constexpr (CDT == fg::kBF16) {
            uint16_t* o = (uint16_t*)a.out + (orow + m) * a.ldo + n;
            if (n + 3 < a.N && (a.ldo & 3) == 0) {
              *(uint2*)o = make_uint2(fg::pack_bf16x2(acc[i][nb][4 * v4], acc[i][nb][4 * v4 + 1]),
                                      fg::pack_bf16x2(acc[i][nb][4 * v4 + 2], acc[i][nb][4 * v4 + 3]));
            } else {
              for (int e = 0; e < 4 && n + e < a.N; ++e) o[e] = fg::f32_to_bf16(acc[i][nb][4 * v4 + e]);
            }
          } else {
            float* o = (float*)a.out + (orow + m) * a.ldo + n;
            if (n + 3 < a.N && (a.ldo & 3) == 0) {
              *(float4*)o = make_float4(acc[i][nb][4 * v4], acc[i][nb][4 * v4 + 1], acc[i][nb][4 * v4 + 2],
                                        acc[i][nb][4 * v4 + 3]);
            } else {
              for (int e = 0; e < 4 && n + e < a.N; ++e) o[e] = acc[i][nb][4 * v4 + e];
            }
          }
        }
      }
    }
    if constexpr (PM) {
      // over the values as stored (rounded to bf16 for a bf16 output)
      if (active) {
#pragma unroll
        for (int i = 0; i < MI; ++i) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int n = n0 + nb * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
            if (n < a.N) {
              const float val =
                  CDT == fg::kBF16 ? fg::bf16_to_f32(fg::f32_to_bf16(acc[i][nb][v])) : acc[i][nb][v];
              pm_max[i] = fmaxf(pm_max[i], val);
              const uint64_t k = fg::rank_key(val, (uint32_t)n);
              pm_key[i] = k > pm_key[i] ? k : pm_key[i];
            }
          }
        }
      }
    }
    if constexpr (KT > 0) {
      // this round's logits (bf16) into LDS: tile[m][32 wave + c], rows of kTileRow bytes
      __syncthreads();  // every wave is done reading the activation stages
      if (lane == 0) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          s_n0[wave * NB + nb] = n0 + nb * 32;
          s_nv[wave * NB + nb] = active ? max(0, min(32, a.N - n0 - nb * 32)) : 0;
        }
      }
      if (active) {
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const int m = i * 32 + l32;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int v4 = 0; v4 < 4; ++v4) {
            const int c = (wave * NB + nb) * 32 + v4 * 8 + g * 4;
            *(uint2*)(smem + m * kTileRow + c * 2) =
                make_uint2(fg::pack_bf16x2(acc[i][nb][4 * v4], acc[i][nb][4 * v4 + 1]),
                           fg::pack_bf16x2(acc[i][nb][4 * v4 + 2], acc[i][nb][4 * v4 + 3]));
          }
        }
      }
      __syncthreads();
      // TPR threads per row scan 8 columns at a time. Keys at or below the row's KT-th best
      // key of the earlier rounds cannot enter its list and are skipped.
      constexpr int TPR = W * 64 / MP;
      const int m = tid / TPR, sub = tid % TPR;
      const bool row_ok = m < a.M && m < MP;
      const uint64_t thr = (row_ok && rd > 0) ? s_keys[m * KT + KT - 1] : 0ull;
      uint64_t top[KT];
#pragma unroll
      for (int i = 0; i < KT; ++i) top[i] = 0;
      fg::LseAcc acc_l{-INFINITY, 0.0f};
      if (row_ok) {
        for (int c = sub * 8; c < 256; c += TPR * 8) {
          const int wv = c >> 5, nv = s_nv[wv];
          if ((c & 31) >= nv) continue;
          const int nbase = s_n0[wv] + (c & 31);
          const uint4 raw = *(const uint4*)(smem + m * kTileRow + c * 2);
          const uint32_t wds[4] = {raw.x, raw.y, raw.z, raw.w};
          float v[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            v[2 * j] = fg::sanitize<SAN>(__uint_as_float(wds[j] << 16));
            v[2 * j + 1] = fg::sanitize<SAN>(__uint_as_float(wds[j] & 0xffff0000u));
          }
          const int valid = min(8, nv - (c & 31));
          float m8 = -INFINITY;
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (j < valid) {
              const uint64_t key = fg::rank_key(v[j], (uint32_t)(nbase + j));
              if (key > thr) fg::insert_key<KT>(top, key);
              m8 = fmaxf(m8, v[j]);
            }
          const float mx = fmaxf(acc_l.m, m8);
          float sm = (acc_l.m == -INFINITY) ? 0.0f : acc_l.s * __expf(acc_l.m - mx);
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (j < valid) sm += __expf(v[j] - mx);
          acc_l = {mx, sm};
        }
      }
      fg::lanes_merge<KT>(top, TPR);
#pragma unroll
      for (int o = TPR / 2; o > 0; o >>= 1) {
        fg::LseAcc other{__shfl_xor(acc_l.m, o, 64), __shfl_xor(acc_l.s, o, 64)};
        acc_l = fg::lse_combine(acc_l, other);
      }
      if (row_ok && sub == 0) {
        if (rd > 0) {
          uint64_t run[KT];
#pragma unroll
          for (int i = 0; i < KT; ++i) run[i] = s_keys[m * KT + i];
          fg::merge_desc<KT>(top, run);
          const float2 p = s_lse[m];
          acc_l = fg::lse_combine(acc_l, fg::LseAcc{p.x, p.y});
        }
#pragma unroll
        for (int i = 0; i < KT; ++i) s_keys[m * KT + i] = top[i];
        s_lse[m] = make_float2(acc_l.m, acc_l.s);
      }
      __syncthreads();  // the tile is read before the next round's activation loads land
    }
  }
  if constexpr (PM) {
    // lane groups 0 and 1 hold the same rows; then the waves' maxima meet in LDS
    __syncthreads();  // every wave is done with the activation stages
    float* s_pmax = (float*)smem;                         // [W][MP]
    uint64_t* s_pkey = (uint64_t*)(smem + W * MP * 4);   // [W][MP]
    static_assert(W * MP * 12 <= kStages * STAGE, "row maxima staging");
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const float mo = __shfl_xor(pm_max[i], 32, 64);
      const uint64_t ko = fg::shfl_xor_u64(pm_key[i], 32);
      if (g == 0) {
        s_pmax[wave * MP + i * 32 + l32] = fmaxf(pm_max[i], mo);
        s_pkey[wave * MP + i * 32 + l32] = ko > pm_key[i] ? ko : pm_key[i];
      }
    }
    __syncthreads();
    for (int m = tid; m < a.M; m += W * 64) {
      float mx = s_pmax[m];
      uint64_t k = s_pkey[m];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        mx = fmaxf(mx, s_pmax[w * MP + m]);
        k = s_pkey[w * MP + m] > k ? s_pkey[w * MP + m] : k;
      }
      a.part_max[(int64_t)m * a.nparts + blockIdx.x] = mx;
      a.part_key[(int64_t)m * a.nparts + blockIdx.x] = k;
    }
  }
  if constexpr (KT > 0) {
    // this workgroup's part of every row
    for (int m = tid; m < a.M; m += W * 64) {
      const int64_t pi = (int64_t)m * a.nparts + blockIdx.x;
#pragma unroll
      for (int i = 0; i < KT; ++i) a.part_keys[pi * KT + i] = s_keys[m * KT + i];
      a.part_lse[pi] = s_lse[m];
    }
  }
}

int g_cus = 0;
std::once_flag g_cus_once;
int device_cus() {
  std::call_once(g_cus_once, [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
      g_cus = n;
    if (g_cus <= 0) g_cus = 256;
  });
  return g_cus;
}

struct Plan {
  int grid, rmax, nparts;
};
Plan plan_for(int N) {
  const int nblk = (N + 31) / 32;
  Plan p;
  p.grid = std::max(1, std::min(device_cus(), (nblk + kBlocks - 1) / kBlocks));
  p.rmax = (nblk + p.grid * kBlocks - 1) / (p.grid * kBlocks);
  p.nparts = p.grid;
  return p;
}
int k_bucket(int kmax) { return kmax <= 1 ? 1 : kmax <= 2 ? 2 : kmax <= 4 ? 4 : kmax <= 8 ? 8 : 16; }

template <int MI, int CDT, int KT, bool SAN, bool PM>
void launch_mi(const LmArgs& a, int grid, hipStream_t s) {
  constexpr int W = waves_for(MI);
  hipLaunchKernelGGL((lm_stream_kernel<MI, CDT, KT, SAN, PM, W>), dim3(grid), dim3(W * 64), 0, s, a);
}
template <int CDT, int KT, bool SAN, bool PM = false>
void launch_rows(const LmArgs& a, int grid, hipStream_t s) {
  if (a.M <= 64) launch_mi<2, CDT, KT, SAN, PM>(a, grid, s);
  else if (a.M <= 128) launch_mi<4, CDT, KT, SAN, PM>(a, grid, s);
  else if (a.M <= 192) launch_mi<6, CDT, KT, SAN, PM>(a, grid, s);
  else if constexpr (KT <= 8) launch_mi<8, CDT, KT, SAN, PM>(a, grid, s);  // (LDS: the host rejects KT 16 here)
}
template <int KT, bool SAN>
void launch_cdt(const LmArgs& a, int out_dtype, int grid, hipStream_t s) {
  if (out_dtype == fg::kF32) launch_rows<fg::kF32, KT, SAN>(a, grid, s);
  else launch_rows<fg::kBF16, KT, SAN>(a, grid, s);
}
template <int KT>
void launch_san(const LmArgs& a, int out_dtype, bool san, int grid, hipStream_t s) {
  if (san) launch_cdt<KT, true>(a, out_dtype, grid, s);
  else launch_cdt<KT, false>(a, out_dtype, grid, s);
}

// ------------------------------------------------------------------ Medusa fc
constexpr int kMedMaxSplit = 8;

struct MedPlan {
  int ngroups, ksplit, grid;
};
// As many key ranges as keep every CU busy with one task (at least 4 k-steps per range).
MedPlan med_plan(int H, int heads) {
  MedPlan p;
  p.ngroups = (H + 32 * kBlocks - 1) / (32 * kBlocks);
  const int base = heads * p.ngroups;
  p.ksplit = std::max(1, std::min({device_cus() / base, H / kKS / 4, kMedMaxSplit}));
  p.grid = std::min(device_cus(), base * p.ksplit);
  return p;
}


// out[h * M + m, n] = R[m, n] + SiLU(sum_p parts[p, h, m, n] + bias[h, n]), 4 columns per thread
// (with bf16 output rounded where the reference's bf16 head rounds: fc + bias, SiLU, sum).
template <int ODT, int RDT>
__global__ void __launch_bounds__(256) medusa_combine_kernel(const float* __restrict__ parts, int ksplit, int heads,
                                                             int M, int N, const uint16_t* __restrict__ bias,
                                                             const void* __restrict__ R, int64_t ldr,
                                                             void* __restrict__ out) {
  const int nq = N >> 2;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)heads * M * nq) return;
  const int c = (int)(idx % nq) * 4;
  const int64_t hm = idx / nq;  // h * M + m
  const int h = (int)(hm / M), m = (int)(hm % M);
  const int64_t plane = (int64_t)heads * M * N;
  float4 pv[kMedMaxSplit];
#pragma unroll
  for (int p = 0; p < kMedMaxSplit; ++p)
    if (p < ksplit) pv[p] = *(const float4*)(parts + p * plane + hm * N + c);
  const uint2 bw = *(const uint2*)(bias + (int64_t)h * N + c);
  float r[4];
  if constexpr (RDT == fg::kBF16) {
    const uint2 rw = *(const uint2*)((const uint16_t*)R + (int64_t)m * ldr + c);
    r[0] = __uint_as_float(rw.x << 16); r[1] = __uint_as_float(rw.x & 0xffff0000u);
    r[2] = __uint_as_float(rw.y << 16); r[3] = __uint_as_float(rw.y & 0xffff0000u);
  } else {
    const float4 rv = *(const float4*)((const float*)R + (int64_t)m * ldr + c);
    r[0] = rv.x; r[1] = rv.y; r[2] = rv.z; r[3] = rv.w;
  }
  float s[4] = {pv[0].x, pv[0].y, pv[0].z, pv[0].w};
#pragma unroll
  for (int p = 1; p < kMedMaxSplit; ++p)
    if (p < ksplit) {
      s[0] += pv[p].x; s[1] += pv[p].y; s[2] += pv[p].z; s[3] += pv[p].w;
    }
  const float b[4] = {__uint_as_float(bw.x << 16), __uint_as_float(bw.x & 0xffff0000u),
                      __uint_as_float(bw.y << 16), __uint_as_float(bw.y & 0xffff0000u)};
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (ODT == fg::kBF16) {
      // the reference's bf16 rounding points (project_hidden under bf16 autocast): the fc output
      // fc(x) + b, SiLU of it, then the residual sum (stored below)
      const float f = fg::round_bf16(s[e] + b[e]);
      v[e] = r[e] + fg::round_bf16(fg::silu_f32(f));
    } else {
      v[e] = r[e] + fg::silu_f32(s[e] + b[e]);
    }
  }
  if constexpr (ODT == fg::kBF16)
    *(uint2*)((uint16_t*)out + hm * N + c) = make_uint2(fg::pack_bf16x2(v[0], v[1]), fg::pack_bf16x2(v[2], v[3]));
  else
    *(float4*)((float*)out + hm * N + c) = make_float4(v[0], v[1], v[2], v[3]);
}

}  // namespace

namespace fg {

bool medusa_stream_ok(int batch, int H, int heads) {
  return batch >= 1 && batch <= 256 && heads >= 1 && H >= kKS && H % kKS == 0 &&
         (uint64_t)heads * H * H * 2 < 0xFFFFFFFFull && (uint64_t)heads * batch * H * 2 < 0xFFFFFFFFull;
}

size_t medusa_stream_parts_bytes(int batch, int H, int heads) {
  return medusa_stream_ok(batch, H, heads) ? (size_t)med_plan(H, heads).ksplit * heads * batch * H * 4 : 0;
}

int medusa_stream(const void* a, int batch, int H, int heads, const void* fc_w, const void* fc_b, const void* R,
                  int64_t ldr, int r_dtype, void* out, int out_dtype, float* parts, hipStream_t s) {
  FG_REQUIRE(medusa_stream_ok(batch, H, heads), "medusa_stream: shape");
  FG_REQUIRE(((uintptr_t)a & 15) == 0 && ((uintptr_t)fc_w & 15) == 0 && ((uintptr_t)parts & 15) == 0 &&
                 ((uintptr_t)fc_b & 7) == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)R & 15) == 0 &&
                 ldr % 4 == 0,
             "medusa_stream: alignment");
  const MedPlan p = med_plan(H, heads);
  LmArgs la{};
  la.x = a; la.ldx = H; la.M = batch; la.K = H;
  la.w = fc_w; la.ldw = H; la.N = H;
  la.out = parts; la.ldo = H;
  la.nparts = p.grid;
  la.heads = heads; la.ksplit = p.ksplit; la.ngroups = p.ngroups;
  la.x_head_bytes = (int64_t)batch * H * 2;
  la.w_head_bytes = (int64_t)H * H * 2;
  if (batch <= 64) hipLaunchKernelGGL((lm_stream_kernel<2, kF32, 0, false, false, 8, true>), dim3(p.grid), dim3(512), 0, s, la);
  else if (batch <= 128) hipLaunchKernelGGL((lm_stream_kernel<4, kF32, 0, false, false, 8, true>), dim3(p.grid), dim3(512), 0, s, la);
  else hipLaunchKernelGGL((lm_stream_kernel<8, kF32, 0, false, false, 8, true>), dim3(p.grid), dim3(512), 0, s, la);
  int rc = check_launch("fg_medusa_heads(stream)");
  if (rc) return rc;
  const int64_t threads = (int64_t)heads * batch * (H / 4);
  const dim3 grid((unsigned)((threads + 255) / 256));
  const uint16_t* bias = (const uint16_t*)fc_b;
  if (out_dtype == kBF16 && r_dtype == kBF16)
    hipLaunchKernelGGL((medusa_combine_kernel<kBF16, kBF16>), grid, dim3(256), 0, s, parts, p.ksplit, heads, batch, H, bias, R, ldr, out);
  else if (out_dtype == kBF16)
    hipLaunchKernelGGL((medusa_combine_kernel<kBF16, kF32>), grid, dim3(256), 0, s, parts, p.ksplit, heads, batch, H, bias, R, ldr, out);
  else if (r_dtype == kBF16)
    hipLaunchKernelGGL((medusa_combine_kernel<kF32, kBF16>), grid, dim3(256), 0, s, parts, p.ksplit, heads, batch, H, bias, R, ldr, out);
  else
    hipLaunchKernelGGL((medusa_combine_kernel<kF32, kF32>), grid, dim3(256), 0, s, parts, p.ksplit, heads, batch, H, bias, R, ldr, out);
  return check_launch("fg_medusa_heads(combine)");
}

}  // namespace fg

extern "C" {

int fg_lm_head_topk_parts(int vocab) { return vocab > 0 ? plan_for(vocab).nparts : 0; }

size_t fg_lm_head_topk_workspace(int rows, int vocab, int kmax) {
  if (rows <= 0 || vocab <= 0 || kmax <= 0) return 256;
  const Plan p = plan_for(vocab);
  return (size_t)rows * p.nparts * (k_bucket(kmax) * sizeof(uint64_t) + sizeof(float2)) + 256;
}

int fg_lm_head_topk(const void* x, int M, int K, int64_t ldx, const int32_t* row_index, const int32_t* row_active,
                    const void* w, int64_t ldw, int N, void* out, int out_dtype, int64_t ldo, int kmax, int sanitize,
                    int32_t* cand_tokens, float* cand_scores, float* row_stats, float* part_max,
                    uint64_t* part_key, void* workspace, size_t workspace_bytes, void* stream) {
  FG_REQUIRE(x && w, "fg_lm_head_topk: null pointer");
  FG_REQUIRE(M >= 1 && M <= 256, "fg_lm_head_topk: M must be in [1, 256]");
  FG_REQUIRE(N >= 1 && K >= kKS && K % kKS == 0, "fg_lm_head_topk: K must be a positive multiple of 64");
  FG_REQUIRE(ldx >= K && ldx % 8 == 0 && ldw >= K && ldw % 8 == 0 && ((uintptr_t)x & 15) == 0 &&
                 ((uintptr_t)w & 15) == 0,
             "fg_lm_head_topk: x and w need 16-byte aligned rows");
  FG_REQUIRE((uint64_t)N * (uint64_t)ldw * 2 <= 0xFFFFFFFFull, "fg_lm_head_topk: w must span less than 4 GiB");
  FG_REQUIRE(out_dtype == fg::kBF16 || out_dtype == fg::kF32, "fg_lm_head_topk: out_dtype");
  FG_REQUIRE(out || kmax > 0, "fg_lm_head_topk: nothing to compute (no out, kmax 0)");
  FG_REQUIRE(!out || ldo >= N, "fg_lm_head_topk: ldo < N");
  // rows whose stride is a multiple of 4 take 4-column vector stores (8 bytes bf16, 16 fp32)
  FG_REQUIRE(!out || ldo % 4 != 0 || ((uintptr_t)out & (out_dtype == fg::kBF16 ? 7 : 15)) == 0,
             "fg_lm_head_topk: out must be aligned to 4 columns when ldo is a multiple of 4");
  FG_REQUIRE(kmax >= 0 && kmax <= 16 && kmax <= N, "fg_lm_head_topk: kmax must be in [0, min(16, N)]");
  FG_REQUIRE(kmax == 0 || (cand_tokens && cand_scores && workspace), "fg_lm_head_topk: candidate outputs missing");
  FG_REQUIRE(kmax == 0 || !row_active, "fg_lm_head_topk: row_active only without top-k");
  FG_REQUIRE(kmax <= 8 || M <= 192, "fg_lm_head_topk: kmax above 8 needs M <= 192");
  FG_REQUIRE(!part_max == !part_key, "fg_lm_head_topk: part_max and part_key go together");
  FG_REQUIRE(!part_max || (kmax == 0 && out), "fg_lm_head_topk: row maxima parts need out and kmax 0");
  const Plan p = plan_for(N);
  LmArgs a{};
  a.x = x; a.ldx = ldx; a.rows = row_index; a.row_active = row_active; a.M = M; a.K = K;
  a.w = w; a.ldw = ldw; a.N = N; a.out = out; a.ldo = ldo;
  a.nparts = p.nparts;
  hipStream_t s = (hipStream_t)stream;
  if (kmax == 0 && part_max) {
    a.part_max = part_max;
    a.part_key = part_key;
    if (out_dtype == fg::kF32) launch_rows<fg::kF32, 0, false, true>(a, p.grid, s);
    else launch_rows<fg::kBF16, 0, false, true>(a, p.grid, s);
    return fg::check_launch("fg_lm_head_topk");
  }
  if (kmax == 0) {
    launch_san<0>(a, out_dtype, false, p.grid, s);
    return fg::check_launch("fg_lm_head_topk");
  }
  const int KB = k_bucket(kmax);
  const size_t need = (size_t)M * p.nparts * (KB * sizeof(uint64_t) + sizeof(float2));
  FG_REQUIRE(workspace_bytes >= need, "fg_lm_head_topk: workspace too small");
  a.part_keys = (uint64_t*)workspace;
  a.part_lse = (float2*)(a.part_keys + (size_t)M * p.nparts * KB);
  const bool san = sanitize != 0;
  switch (KB) {
    case 1: launch_san<1>(a, out_dtype, san, p.grid, s); break;
    case 2: launch_san<2>(a, out_dtype, san, p.grid, s); break;
    case 4: launch_san<4>(a, out_dtype, san, p.grid, s); break;
    case 8: launch_san<8>(a, out_dtype, san, p.grid, s); break;
    default: launch_san<16>(a, out_dtype, san, p.grid, s); break;
  }
  int rc = fg::check_launch("fg_lm_head_topk");
  if (rc) return rc;
  return fg::topk_merge_parts(KB, a.part_keys, a.part_lse, M, p.nparts, kmax, cand_tokens, cand_scores, row_stats, s);
}

}  // extern "C"
