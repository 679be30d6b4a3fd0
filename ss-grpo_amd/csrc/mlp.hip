// The decoder layer's MLP input projection with its activation fused into the GEMM epilogue:
//
//   out[M, I] = bf16(silu(bf16(x . Wg^T))) * bf16(x . Wu^T)        W = [Wg; Wu], the [2I, H] gate_up weight
//
// bf16 operands, fp32 accumulation; gate and up are rounded to bf16 before the activation and
// SiLU(gate) before the product, as the unfused projection + `fg_swiglu` (and the Hugging Face
// MLP the reference runs under bf16 autocast) round them, so the result equals that pair's
// whenever the two GEMMs' fp32 sums round to the same bf16 values.
// The [M, 2I] gate/up intermediate is never written.
//
// Replaces `act_fn(gate_proj(x)) * up_proj(x)` of the Hugging Face Qwen2/Llama MLP inside each
// decoder layer of the reference's tree-verify forward (flashgrpo/models/qwen_flashgrpo_wrapper.py:
// 172-180 runs the HF decoder layers).
//
// Tiling (gfx950): one workgroup of 4 waves (2 x 2, one per SIMD) per output tile of BM rows x 128
// intermediate columns (BM = 64, 128, 192 or 256). The tile's 256 weight rows sit in LDS as
// [gate 64 | up 64 | gate 64 | up 64], so the wave that owns output columns c .. c+63 holds both
// the gate and the up accumulators of those columns and applies the activation in registers.
// K advances 64 per step through an NS-stage LDS ring (the deepest that fits 160 KB: 4 stages for
// 64-row tiles, 3 for 128, 2 for 192 and 256) filled by direct HBM->LDS buffer loads
// (`buffer_load_dwordx4 ... lds`, 1 KB = 8 rows per instruction), rows of 128 bytes with the
// 16-byte chunks XOR-swizzled by row so that the fragment reads of 32 consecutive rows hit
// distinct banks. Each k-step is four k16 sub-steps of v_mfma_f32_32x32x16_bf16 (the wave's
// (BM/2) x 128 block is (BM/64) x 4 MFMA tiles, computed transposed so each lane ends with 4
// consecutive output columns of one row); the fragment reads of sub-step s+1 are interleaved with
// the MFMAs of sub-step s, and the loads of k-step t+NS are issued between the MFMAs of k-step t's
// last sub-step, after the one barrier of the step. The output block of each wave goes out
// through LDS as whole 128-byte row segments.
// Workgroups are numbered so that each XCD takes a contiguous run of tiles along M for one weight
// stripe: the stripe is read from HBM once per XCD and reused from its L2. Which tile height (or
// the library projection + fg_swiglu) is fastest depends on the shape; the caller decides from
// measurements.
#include "fg_common.h"

#include <type_traits>

#include <algorithm>


namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kBK = 64;          // K per step
constexpr int kRowBytes = 128;   // one LDS row: kBK bf16
constexpr int kSub = kBK / 16;   // k16 MFMA sub-steps per step
constexpr int kBN = 256;         // weight rows per tile (128 gate + 128 up)
constexpr int kCols = kBN / 2;   // output columns per tile

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


struct MlpArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* w;  // [2 * inter, ldw]: gate rows, then up rows
  int64_t ldw;
  uint16_t* out;
  int64_t ldo;
  int rows, inter, hidden;
  int vec16;  // out rows 16-byte aligned: whole 8-column chunks as one store
  int tiles_m, tiles, per_xcd;
};

// Ring depth of a BM-row tile: as many k-steps as fit the CU's 160 KB of LDS, at most 4.
constexpr int stages_for(int bm) { return std::min(4, (160 * 1024) / ((bm + kBN) * kRowBytes)); }

template <int BM>
__global__ void __launch_bounds__(256, 1) gate_up_swiglu_kernel(MlpArgs p) {
  constexpr int NS = stages_for(BM);
  constexpr int WM = BM / 2;                       // rows per wave
  constexpr int FM = WM / 32, FN = 4;              // MFMA tiles per wave: rows x (2 gate + 2 up)
  constexpr int A_BYTES = BM * kRowBytes, B_BYTES = kBN * kRowBytes, STAGE = A_BYTES + B_BYTES;
  constexpr int LA = A_BYTES / 4096, LB = B_BYTES / 4096, LPW = LA + LB;  // 1 KB loads per wave per step
  static_assert(LA * 4096 == A_BYTES && LB == 8, "each wave loads BM/4 x-rows and one 64-row weight block");
  static_assert(FM * FN <= LPW, "the loads of a step are spread over the last sub-step's MFMAs");
  static_assert(NS >= 2 && NS * STAGE <= 160 * 1024 && (NS - 1) * LPW < 64, "ring stages: LDS and vmcnt");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * STAGE];

  // XCD-aware tile order: workgroup b runs on XCD b % 8; XCD x takes tiles x*per_xcd .. +per_xcd-1,
  // which walk down M for one weight stripe before the next stripe.
  const int xcd = blockIdx.x % 8, j = blockIdx.x / 8;
  const int tile = xcd * p.per_xcd + j;
  if (j >= p.per_xcd || tile >= p.tiles) return;  // whole workgroup: before any barrier
  const int m0 = (tile % p.tiles_m) * BM, c0 = (tile / p.tiles_m) * kCols;
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, half = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;

  // Buffer descriptors: rows past the matrix end read as zero (rows >= p.rows, columns >= inter).
  const int64_t x_bytes = (int64_t)(p.rows - m0) * p.ldx * 2;
  const int64_t w_bytes = (int64_t)(p.inter - c0) * p.ldw * 2;
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x + (int64_t)m0 * p.ldx), (short)0, (int)(x_bytes < 0x7fffffff ? x_bytes : 0x7fffffff), 0x00020000);
  // wave w fills LDS weight block w: gate rows (w even) or up rows (w odd) c0 + (w / 2) * 64 ..
  const uint16_t* wblock = p.w + ((wave & 1) ? (int64_t)p.inter : 0) * p.ldw + (int64_t)c0 * p.ldw;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)wblock, (short)0, (int)(w_bytes < 0x7fffffff ? w_bytes : 0x7fffffff), 0x00020000);

  // Load lanes: lane l writes LDS bytes l*16 .. of its 1 KB, i.e. row l/8, stored chunk l%8, which
  // holds the row's logical chunk (l%8) ^ (row%8).
  const int lrow = lane >> 3;
  const int lchunk = (lane & 7) ^ (lrow & 7);
  uint32_t xoff[LA], woff[LB];
#pragma unroll
  for (int u = 0; u < LA; ++u) xoff[u] = (uint32_t)(((wave * LA + u) * 8 + lrow) * p.ldx * 2 + lchunk * 16);
#pragma unroll
  for (int u = 0; u < LB; ++u) woff[u] = (uint32_t)((((wave >> 1) * LB + u) * 8 + lrow) * p.ldw * 2 + lchunk * 16);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;
  const int nk = p.hidden / kBK;

  // One 1 KB HBM->LDS load (q < LA: x rows, else weight rows) of k-step ks into ring slot `slot`.
  // M0 holds the LDS address; the s_nop covers the M0-write -> LDS-DMA hazard.
  auto issue = [&](int ks, int slot, int q) __attribute__((always_inline)) {
    const uint32_t koff = (uint32_t)ks * (kBK * 2);
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
      rb[buf][f] = *(const bf16x8*)(st + A_BYTES + frag[s] + (wn * 128 + f * 32) * kRowBytes);
  };
  // One sub-step's MFMAs, the next sub-step's fragment reads placed between them.
  auto mfma_step = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int k = 0; k < FM; ++k)
        acc[i][k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rb[buf][i], ra[buf][k], acc[i][k], 0, 0, 0);
#pragma unroll
    for (int q = 0; q < FM + FN; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - (FM + FN), 0);
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
          __builtin_amdgcn_sched_barrier(0);
          issue(t + NS, slot, i * FM + k);
          __builtin_amdgcn_sched_barrier(0);
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
  wait_vmcnt<0>();  // (the last step already waited for every load)

  // Epilogue: acc[i] (gate) and acc[i + 2] (up) hold the same 4 output columns of one row per lane
  // (32 rows per store instruction). After the last step's barrier no wave reads the ring and no load
  // is in flight, so each wave stages its own (BM/2) x 64 bf16 block in LDS (rows of 128 bytes, 16-byte
  // chunk q of row r stored at chunk q ^ (r % 8)) and writes it back as whole 128-byte row segments.
  unsigned char* stage = smem + wave * (WM * 128);
#pragma unroll
  for (int k = 0; k < FM; ++k)
#pragma unroll
    for (int i = 0; i < FN / 2; ++i)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gt = fg::round_bf16(acc[i][k][4 * v4 + e]), up = fg::round_bf16(acc[i + FN / 2][k][4 * v4 + e]);
          o[e] = fg::round_bf16(fg::silu_f32(gt)) * up;  // the expression of fg_swiglu (bf16)
        }
        const int r = k * 32 + l32, q = i * 4 + v4;
        *(uint2*)(stage + r * 128 + ((q ^ (r & 7)) * 16) + half * 8) =
            make_uint2(fg::pack_bf16x2(o[0], o[1]), fg::pack_bf16x2(o[2], o[3]));
      }
  const int cw = c0 + wn * 64;
#pragma unroll
  for (int it = 0; it < WM / 8; ++it) {
    const int r = it * 8 + (lane >> 3), q = lane & 7;
    const uint4 v = *(const uint4*)(stage + r * 128 + ((q ^ (r & 7)) * 16));
    const int m = m0 + wm * WM + r, c = cw + q * 8;
    if (m >= p.rows || c >= p.inter) continue;
    uint16_t* dst = p.out + (int64_t)m * p.ldo + c;
    if (p.vec16 && c + 8 <= p.inter) {
      *(uint4*)dst = v;
    } else {
      *(uint2*)dst = make_uint2(v.x, v.y);
      if (c + 4 < p.inter) *(uint2*)(dst + 4) = make_uint2(v.z, v.w);
    }
  }
}

template <int BM>
void launch(MlpArgs p, hipStream_t s) {
  p.tiles_m = (p.rows + BM - 1) / BM;
  p.tiles = p.tiles_m * ((p.inter + kCols - 1) / kCols);
  p.per_xcd = (p.tiles + 7) / 8;
  hipLaunchKernelGGL(gate_up_swiglu_kernel<BM>, dim3(8 * p.per_xcd), dim3(256), 0, s, p);
}

// Tile height when the caller leaves it open: of 192 and 256, the one with the fewer MFMA
// row-blocks over whole waves of 256 concurrent tiles (one per CU); ties go to 256 rows (more
// MFMAs per LDS byte). The 64- and 128-row tiles are taken when a caller's measurement asks.
int pick_tile_rows(int rows, int inter) {
  const int64_t cols = (inter + kCols - 1) / kCols;
  auto cost = [&](int bm) { return ((((rows + bm - 1) / bm) * cols + 255) / 256) * bm; };
  return cost(192) < cost(256) ? 192 : 256;
}

}  // namespace

extern "C" {

int fg_gate_up_swiglu(const void* x, int64_t ldx, const void* w_gate_up, int64_t ldw, void* out, int64_t ldo, int rows,
                      int inter, int hidden, int tile_rows, void* stream) {
  FG_REQUIRE(x && w_gate_up && out, "fg_gate_up_swiglu: null pointer");
  FG_REQUIRE(rows > 0 && rows <= (1 << 24) && inter > 0 && hidden > 0, "fg_gate_up_swiglu: bad shape");
  FG_REQUIRE(hidden % kBK == 0, "fg_gate_up_swiglu: hidden size must be a multiple of 64");
  FG_REQUIRE(inter % 4 == 0, "fg_gate_up_swiglu: intermediate size must be a multiple of 4");
  FG_REQUIRE(ldx >= hidden && ldw >= hidden && ldo >= inter && ldx < (1 << 22) && ldw < (1 << 22),
             "fg_gate_up_swiglu: bad row strides");
  FG_REQUIRE(ldx % 8 == 0 && ldw % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w_gate_up & 15) == 0,
             "fg_gate_up_swiglu: x and weight rows must start 16-byte aligned");
  FG_REQUIRE(ldo % 4 == 0 && ((uintptr_t)out & 7) == 0, "fg_gate_up_swiglu: out rows must start 8-byte aligned");
  FG_REQUIRE(tile_rows == 0 || tile_rows == 64 || tile_rows == 128 || tile_rows == 192 || tile_rows == 256,
             "fg_gate_up_swiglu: tile_rows must be 0, 64, 128, 192 or 256");
  FG_REQUIRE((int64_t)((rows + 63) / 64) * ((inter + kCols - 1) / kCols) < (1 << 30), "fg_gate_up_swiglu: too many tiles");
  MlpArgs p{};
  p.x = (const uint16_t*)x;
  p.ldx = ldx;
  p.w = (const uint16_t*)w_gate_up;
  p.ldw = ldw;
  p.out = (uint16_t*)out;
  p.ldo = ldo;
  p.rows = rows;
  p.inter = inter;
  p.hidden = hidden;
  p.vec16 = ldo % 8 == 0 && ((uintptr_t)out & 15) == 0;
  hipStream_t s = (hipStream_t)stream;
  switch (tile_rows ? tile_rows : pick_tile_rows(rows, inter)) {
    case 64: launch<64>(p, s); break;
    case 128: launch<128>(p, s); break;
    case 192: launch<192>(p, s); break;
    default: launch<256>(p, s); break;
  }
  return fg::check_launch("fg_gate_up_swiglu");
}

}  // extern "C"
