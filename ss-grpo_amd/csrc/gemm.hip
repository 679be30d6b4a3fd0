// Dense contractions of the rollout step: the tied LM-head projection and the
// Medusa residual block.
//
//   C[M, N] = epilogue(A[M, K] . B[N, K]^T)      (both operands K-contiguous)
//
// bf16 path: MFMA v_mfma_f32_32x32x16_bf16 tiles, LDS double buffering, fp32
// accumulation, XCD-aware block order (consecutive tiles of one N column
// stripe land on the same XCD so the weight stripe is read from HBM once and
// reused from that XCD's L2 across the M tiles). fp32 path: LDS-tiled FMA
// kernel used by the fp32 configuration.
//
// Replaces the lm_head calls of flashgrpo/decoding/flash_medusa_decoder.py:289-294,
// 414-433, 1079-1091 and MedusaPredictionHead.project_hidden
// (flashgrpo/models/medusa_heads.py:74-78).
#include "fg_common.h"
#include "fg_stream.h"

#include <algorithm>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));  // 16-byte register value (no struct copies)
typedef float floatx4 __attribute__((ext_vector_type(4)));

enum Epilogue : int { kEpiNone = 0, kEpiMedusa = 1 };

struct GemmArgs {
  const void* A;
  int64_t lda;
  int64_t a_batch;
  const int32_t* a_rows;  // optional row gather for A
  const int32_t* row_active;  // optional: tiles whose rows are all 0 here are skipped
  const void* B;
  int64_t ldb;
  int64_t b_batch;
  void* C;
  int64_t ldc;
  int64_t c_batch;
  const void* bias;       // medusa: [N] per batch (dtype of B)
  int64_t bias_batch;
  const void* R;          // medusa residual [M, N] (dtype r_dtype)
  int64_t ldr;
  int64_t r_batch;
  int r_dtype;
  int M, N, K;
};


// Block-uniform: does any row of [m0, m0 + rows) have a non-zero row_active flag?
FG_DEVICE bool tile_has_active_row(const GemmArgs& g, int m0, int rows) {
  int any = 0;
  for (int r = threadIdx.x; r < rows; r += blockDim.x)
    if (m0 + r < g.M) any |= g.row_active[m0 + r] != 0;
  return __syncthreads_or(any) != 0;
}

template <int CDT, int BDT>
FG_DEVICE void epilogue_store(const GemmArgs& g, int z, int m, int n, float acc, int epi) {
  if (m >= g.M || n >= g.N) return;
  float v = acc;
  if (epi == kEpiMedusa) {
    float b = fg::load_elem<BDT>(g.bias, z * g.bias_batch + n);
    float r = g.r_dtype == fg::kBF16 ? fg::load_elem<fg::kBF16>(g.R, z * g.r_batch + (int64_t)m * g.ldr + n)
                                     : fg::load_elem<fg::kF32>(g.R, z * g.r_batch + (int64_t)m * g.ldr + n);
    if constexpr (CDT == fg::kBF16) {
      // the reference's bf16 rounding points: fc(x) + b, SiLU of it, then the residual sum
      const float f = fg::round_bf16(v + b);
      v = r + fg::round_bf16(fg::silu_f32(f));
    } else {
      v = r + fg::silu_f32(v + b);
    }
  }
  fg::store_elem<CDT>(g.C, z * g.c_batch + (int64_t)m * g.ldc + n, v);
}

// ----------------------------------------------------------------- bf16 MFMA
constexpr int kBK = 64;
constexpr int kPad = 8;  // bf16 elements of padding per LDS row (16 bytes)
constexpr int kLdsRow = kBK + kPad;

// Row of accumulator element i held by `lane` in a 32x32 MFMA output tile.
FG_DEVICE int c_row32(int i, int lane) { return (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3); }

template <int BM, int BN, int WM, int WN, int CDT>
__global__ void __launch_bounds__(256) gemm_bf16_kernel(GemmArgs g, int epi, int tiles_m, int tiles_n) {
  constexpr int WAVES_N = BN / WN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_CHUNKS = BM * kBK / 8 / 256;  // 16-byte chunks per thread
  constexpr int B_CHUNKS = BN * kBK / 8 / 256;
  static_assert((BM / WM) * (BN / WN) == 4, "4 waves");
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * kLdsRow];

  // XCD-aware tile order: blocks are dispatched round-robin over 8 XCDs; give
  // each XCD a contiguous range of tiles, M fastest, so an N stripe of the
  // weight is shared by tiles resident on one XCD.
  const int nblocks = tiles_m * tiles_n;
  const int bid = blockIdx.x;
  const int q = nblocks / 8, rem = nblocks % 8;
  const int xcd = bid % 8, local = bid / 8;
  const int t = xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
  const int tm = t % tiles_m, tn = t / tiles_m;
  const int z = blockIdx.z;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (g.row_active && !tile_has_active_row(g, m0, BM)) return;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  const uint16_t* Ab = (const uint16_t*)g.A + z * g.a_batch;
  const uint16_t* Bb = (const uint16_t*)g.B + z * g.b_batch;

  // Per-thread global source rows (fixed across k tiles).
  const uint16_t* a_src[A_CHUNKS];
  int a_dst[A_CHUNKS];
#pragma unroll
  for (int c = 0; c < A_CHUNKS; ++c) {
    int idx = tid + c * 256;
    int r = idx / (kBK / 8), col = (idx % (kBK / 8)) * 8;
    int m = min(m0 + r, g.M - 1);
    int src_row = g.a_rows ? g.a_rows[m] : m;
    a_src[c] = Ab + (int64_t)src_row * g.lda + col;
    a_dst[c] = r * kLdsRow + col;
  }
  const uint16_t* b_src[B_CHUNKS];
  int b_dst[B_CHUNKS];
#pragma unroll
  for (int c = 0; c < B_CHUNKS; ++c) {
    int idx = tid + c * 256;
    int r = idx / (kBK / 8), col = (idx % (kBK / 8)) * 8;
    int n = min(n0 + r, g.N - 1);
    b_src[c] = Bb + (int64_t)n * g.ldb + col;
    b_dst[c] = r * kLdsRow + col;
  }

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  uint4 ra[A_CHUNKS], rb[B_CHUNKS];
  const int ktiles = g.K / kBK;
  // prologue
#pragma unroll
  for (int c = 0; c < A_CHUNKS; ++c) ra[c] = *(const uint4*)(a_src[c]);
#pragma unroll
  for (int c = 0; c < B_CHUNKS; ++c) rb[c] = *(const uint4*)(b_src[c]);
#pragma unroll
  for (int c = 0; c < A_CHUNKS; ++c) *(uint4*)&As[0][a_dst[c]] = ra[c];
#pragma unroll
  for (int c = 0; c < B_CHUNKS; ++c) *(uint4*)&Bs[0][b_dst[c]] = rb[c];
  __syncthreads();

  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) {
      const int koff = (kt + 1) * kBK;
#pragma unroll
      for (int c = 0; c < A_CHUNKS; ++c) ra[c] = *(const uint4*)(a_src[c] + koff);
#pragma unroll
      for (int c = 0; c < B_CHUNKS; ++c) rb[c] = *(const uint4*)(b_src[c] + koff);
    }
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      bf16x8 af[TM], bfr[TN];
      const int kcol = kk * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        int r = wm * WM + i * 32 + (lane & 31);
        af[i] = *(const bf16x8*)&As[cur][r * kLdsRow + kcol];
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        int r = wn * WN + j * 32 + (lane & 31);
        bfr[j] = *(const bf16x8*)&Bs[cur][r * kLdsRow + kcol];
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
#pragma unroll
      for (int c = 0; c < A_CHUNKS; ++c) *(uint4*)&As[cur ^ 1][a_dst[c]] = ra[c];
#pragma unroll
      for (int c = 0; c < B_CHUNKS; ++c) *(uint4*)&Bs[cur ^ 1][b_dst[c]] = rb[c];
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        int m = m0 + wm * WM + i * 32 + c_row32(v, lane);
        int n = n0 + wn * WN + j * 32 + (lane & 31);
        epilogue_store<CDT, fg::kBF16>(g, z, m, n, acc[i][j][v], epi);
      }
}

// ----------------------------------------------------------------- bf16 MFMA, 256-wide N tiles
// Block tile BM x 256 x 64, 4 waves as 2 (M) x 2 (N), wave tile (BM/2) x 128.
// The MFMA is issued with the B fragment as its first operand, so every
// 32x32 accumulator is a tile of C^T: lane l holds row m = l % 32 of C and,
// for each group of 4 accumulator registers, 4 consecutive columns -- the
// epilogue writes 8-byte (bf16) / 16-byte (fp32) runs instead of scalars.
// LDS rows are padded to 72 elements (144 B), which keeps the 16-byte
// fragment reads of 16 consecutive rows on distinct banks.
template <int BM, int CDT>
__global__ void __launch_bounds__(256) gemm_bf16_wide_kernel(GemmArgs g, int epi, int tiles_m, int tiles_n) {
  constexpr int BN = 256;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_CHUNKS = BM * kBK / 8 / 256;
  constexpr int B_CHUNKS = BN * kBK / 8 / 256;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * kLdsRow];

  const int nblocks = tiles_m * tiles_n;
  const int bid = blockIdx.x;
  const int q = nblocks / 8, rem = nblocks % 8;
  const int xcd = bid % 8, local = bid / 8;
  const int t = xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
  const int tm = t % tiles_m, tn = t / tiles_m;
  const int z = blockIdx.z;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (g.row_active && !tile_has_active_row(g, m0, BM)) return;
  const int wm = wave >> 1, wn = wave & 1;

  const uint16_t* Ab = (const uint16_t*)g.A + z * g.a_batch;
  const uint16_t* Bb = (const uint16_t*)g.B + z * g.b_batch;
  const uint16_t* a_src[A_CHUNKS];
  int a_dst[A_CHUNKS];
#pragma unroll
  for (int c = 0; c < A_CHUNKS; ++c) {
    int idx = tid + c * 256;
    int r = idx >> 3, col = (idx & 7) * 8;
    int m = min(m0 + r, g.M - 1);
    int src_row = g.a_rows ? g.a_rows[m] : m;
    a_src[c] = Ab + (int64_t)src_row * g.lda + col;
    a_dst[c] = r * kLdsRow + col;
  }
  const uint16_t* b_src[B_CHUNKS];
  int b_dst[B_CHUNKS];
#pragma unroll
  for (int c = 0; c < B_CHUNKS; ++c) {
    int idx = tid + c * 256;
    int r = idx >> 3, col = (idx & 7) * 8;
    int n = min(n0 + r, g.N - 1);
    b_src[c] = Bb + (int64_t)n * g.ldb + col;
    b_dst[c] = r * kLdsRow + col;
  }

  floatx16 acc[TN][TM];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[j][i][v] = 0.0f;

  uint4 ra[A_CHUNKS], rb[B_CHUNKS];
  const int ktiles = g.K / kBK;
#pragma unroll
  for (int c = 0; c < A_CHUNKS; ++c) ra[c] = *(const uint4*)(a_src[c]);
#pragma unroll
  for (int c = 0; c < B_CHUNKS; ++c) rb[c] = *(const uint4*)(b_src[c]);
#pragma unroll
  for (int c = 0; c < A_CHUNKS; ++c) *(uint4*)&As[0][a_dst[c]] = ra[c];
#pragma unroll
  for (int c = 0; c < B_CHUNKS; ++c) *(uint4*)&Bs[0][b_dst[c]] = rb[c];
  __syncthreads();

  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) {
      const int koff = (kt + 1) * kBK;
#pragma unroll
      for (int c = 0; c < A_CHUNKS; ++c) ra[c] = *(const uint4*)(a_src[c] + koff);
#pragma unroll
      for (int c = 0; c < B_CHUNKS; ++c) rb[c] = *(const uint4*)(b_src[c] + koff);
    }
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int kcol = kk * 16 + (lane >> 5) * 8;
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *(const bf16x8*)&As[cur][(wm * WM + i * 32 + (lane & 31)) * kLdsRow + kcol];
#pragma unroll
      for (int j = 0; j < TN; ++j) bfr[j] = *(const bf16x8*)&Bs[cur][(wn * WN + j * 32 + (lane & 31)) * kLdsRow + kcol];
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[j][i], 0, 0, 0);
    }
    if (more) {
#pragma unroll
      for (int c = 0; c < A_CHUNKS; ++c) *(uint4*)&As[cur ^ 1][a_dst[c]] = ra[c];
#pragma unroll
      for (int c = 0; c < B_CHUNKS; ++c) *(uint4*)&Bs[cur ^ 1][b_dst[c]] = rb[c];
    }
    __syncthreads();
  }

  // Epilogue: acc[j][i] is the C^T tile (n rows, m columns) -> lane owns row m.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * WM + i * 32 + (lane & 31);
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const int n = n0 + wn * WN + j * 32 + v4 * 8 + (lane >> 5) * 4;
        float o[4] = {acc[j][i][4 * v4], acc[j][i][4 * v4 + 1], acc[j][i][4 * v4 + 2], acc[j][i][4 * v4 + 3]};
        if (epi == kEpiNone && n + 3 < g.N) {
          if constexpr (CDT == fg::kBF16) {
            uint32_t w0 = (uint32_t)fg::f32_to_bf16(o[0]) | ((uint32_t)fg::f32_to_bf16(o[1]) << 16);
            uint32_t w1 = (uint32_t)fg::f32_to_bf16(o[2]) | ((uint32_t)fg::f32_to_bf16(o[3]) << 16);
            *(uint2*)((uint16_t*)g.C + z * g.c_batch + (int64_t)m * g.ldc + n) = make_uint2(w0, w1);
          } else {
            *(float4*)((float*)g.C + z * g.c_batch + (int64_t)m * g.ldc + n) = make_float4(o[0], o[1], o[2], o[3]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) epilogue_store<CDT, fg::kBF16>(g, z, m, n + e, o[e], epi);
        }
      }
  }
}

// ----------------------------------------------------------------- bf16 weight streaming, M <= 256
// For the skinny products of the rollout (LM head over <= 256 rows, Medusa fc
// over the batch) the weight matrix B is read exactly once and dominates the
// bytes, so B never goes through LDS: every wave owns 16 rows of B and streams
// them from global memory straight into registers with v_mfma_f32_16x16x32_bf16
// operand layout. Per 128-wide k-tile, lane (n, q) = (l % 16, l / 16) holds the
// 64 contiguous bytes B[n][k0 + q*32 .. +32]: each row is read as 256-byte runs
// by four lanes (the access pattern that measured fastest for this stream).
// A (<= 256 rows) is staged per k-tile in LDS (double-buffered) and shared by
// all waves of the workgroup; its 16-byte pieces are XOR-swizzled by row & 15,
// which keeps the fragment reads free of bank conflicts without padding.
//
// Loads run PF k-tiles ahead in register rings (A staging chunks first, then
// the W pieces of the same tile). Every load is issued unconditionally (past the
// last k-tile they re-read one fixed line) so the wait counts stay static:
// consuming tile kt waits only for the loads of tile kt, not for younger ones.
//
// k order inside a k-tile: MFMA step s uses piece s (8 k) of each lane's 32-k
// run, i.e. k = k0 + q*32 + s*8 + j for the lane group q; the A fragments read
// the same k's, so the products sum the same terms as the natural order. Each
// 16x16 accumulator is a tile of C^T (lane owns column m = l % 16 and rows
// n = 4*(l/16) .. +4), so the epilogue writes 4 consecutive n per store.
constexpr int kST = 128;  // k-tile of the streaming kernel
FG_DEVICE int a_swz16(int row, int piece) { return row * kST + ((piece ^ (row & 15)) << 3); }

// Up to 32 rows of A the kernel fits in 128 VGPRs, so two workgroups share a CU
// (more loads in flight per CU).
constexpr int stream_occupancy(int mb) { return mb <= 2 ? 2 : 1; }

template <int MB, int WAVES, int PF, int CDT>
__global__ void __launch_bounds__(WAVES * 64, stream_occupancy(MB) * WAVES / 4) gemm_bf16_stream_kernel(GemmArgs g,
                                                                                                       int epi) {
  constexpr int NT = WAVES * 64;
  constexpr int MROWS = MB * 16;
  constexpr int AC = MROWS * (kST / 8) / NT;  // A staging chunks per thread
  static_assert(AC >= 1 && MROWS * (kST / 8) % NT == 0, "A staging split");
  static_assert(PF == 4 || PF == 2, "the ring below is written out for four or two slots");
  __shared__ __attribute__((aligned(16))) uint16_t As[2][MROWS * kST];
  // (kST-wide k-tiles, MROWS <= 128)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q4 = lane >> 4;
  const int z = blockIdx.y;
  const int n_base = blockIdx.x * (WAVES * 16) + wave * 16;
  if (g.row_active && !tile_has_active_row(g, 0, g.M)) return;

  const uint16_t* Ab = (const uint16_t*)g.A + z * g.a_batch;
  const uint16_t* Bb = (const uint16_t*)g.B + z * g.b_batch;
  const v4u* dummy = (const v4u*)Bb;  // target of the loads past the last k-tile
  // This lane's B row (clamped for loads; rows >= N are not stored).
  const int nb = min(n_base + (lane & 15), g.N - 1);
  const uint16_t* bsrc = Bb + (int64_t)nb * g.ldb + q4 * 32;
  // A staging: chunk c of thread t is row (t + c*NT) / 16, 16-byte piece (t % 16).
  const uint16_t* a_src = Ab + (tid & 15) * 8;
  int64_t a_off[AC];
  int a_dst[AC];
#pragma unroll
  for (int c = 0; c < AC; ++c) {
    int idx = tid + c * NT;
    int r = idx >> 4;
    int m = min(r, g.M - 1);
    int src_row = g.a_rows ? g.a_rows[m] : m;
    a_off[c] = (int64_t)src_row * g.lda;
    a_dst[c] = a_swz16(r, idx & 15);
  }

  floatx4 acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  const int ktiles = g.K / kST;  // a multiple of PF (host check)
  // Ring slots as separate named arrays (constant indices only) so they stay in VGPRs.
  v4u w0[4], w1[4], w2[4], w3[4], a0[AC], a1[AC], a2[AC], a3[AC];
#define FG_ISSUE(W, A, KT)                                                                                  \
  {                                                                                                         \
    const int kt_ = (KT);                                                                                   \
    const bool live_ = kt_ < ktiles;                                                                        \
    _Pragma("unroll") for (int c = 0; c < AC; ++c) A[c] = live_ ? *(const v4u*)(a_src + a_off[c] + kt_ * kST) : *dummy; \
    _Pragma("unroll") for (int p = 0; p < 4; ++p) W[p] = live_ ? *(const v4u*)(bsrc + kt_ * kST + p * 8) : *dummy; \
  }
#define FG_STEP(W, A_NEXT, U)                                                                               \
  {                                                                                                         \
    const int cur = (kt0 + (U)) & 1;                                                                        \
    _Pragma("unroll") for (int st = 0; st < 4; ++st) {                                                      \
      const bf16x8 wf = __builtin_bit_cast(bf16x8, W[st]);                                                  \
      _Pragma("unroll") for (int i = 0; i < MB; ++i) {                                                      \
        const bf16x8 af = *(const bf16x8*)&As[cur][a_swz16(i * 16 + (lane & 15), q4 * 4 + st)];             \
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, af, acc[i], 0, 0, 0);                          \
      }                                                                                                     \
    }                                                                                                       \
    _Pragma("unroll") for (int c = 0; c < AC; ++c) *(v4u*)&As[cur ^ 1][a_dst[c]] = A_NEXT[c];             \
  }
  FG_ISSUE(w0, a0, 0)
  FG_ISSUE(w1, a1, 1)
  if constexpr (PF == 4) {
    FG_ISSUE(w2, a2, 2)
    FG_ISSUE(w3, a3, 3)
  }
#pragma unroll
  for (int c = 0; c < AC; ++c) *(v4u*)&As[0][a_dst[c]] = a0[c];
  __syncthreads();

  for (int kt0 = 0; kt0 < ktiles; kt0 += PF) {
    // step u consumes slot u, stores the A tile of slot u+1, refills slot u with tile kt0+u+PF
    if constexpr (PF == 4) {
      FG_STEP(w0, a1, 0) FG_ISSUE(w0, a0, kt0 + 4) __syncthreads();
      FG_STEP(w1, a2, 1) FG_ISSUE(w1, a1, kt0 + 5) __syncthreads();
      FG_STEP(w2, a3, 2) FG_ISSUE(w2, a2, kt0 + 6) __syncthreads();
      FG_STEP(w3, a0, 3) FG_ISSUE(w3, a3, kt0 + 7) __syncthreads();
    } else {
      FG_STEP(w0, a1, 0) FG_ISSUE(w0, a0, kt0 + 2) __syncthreads();
      FG_STEP(w1, a0, 1) FG_ISSUE(w1, a1, kt0 + 3) __syncthreads();
    }
  }
#undef FG_ISSUE
#undef FG_STEP

  // Epilogue: acc[i] is the C^T tile (16 n rows, 16 m columns) -> lane owns column m.
  const int n = n_base + q4 * 4;
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    const int m = i * 16 + (lane & 15);
    if (m >= g.M) continue;
    float o[4] = {acc[i][0], acc[i][1], acc[i][2], acc[i][3]};
    if (epi == kEpiNone && n + 3 < g.N && (g.ldc & 3) == 0) {
      if constexpr (CDT == fg::kBF16) {
        *(uint2*)((uint16_t*)g.C + z * g.c_batch + (int64_t)m * g.ldc + n) =
            make_uint2(fg::pack_bf16x2(o[0], o[1]), fg::pack_bf16x2(o[2], o[3]));
      } else {
        *(float4*)((float*)g.C + z * g.c_batch + (int64_t)m * g.ldc + n) = make_float4(o[0], o[1], o[2], o[3]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) epilogue_store<CDT, fg::kBF16>(g, z, m, n + e, o[e], epi);
    }
  }
}

// 129..256 rows of A: the same stream with v_mfma_f32_32x32x16_bf16 and 32 rows
// of B per wave, which halves the LDS reads of A per byte of B (at this M the
// A fragment reads, not HBM, would otherwise bound the kernel). 64-wide k-tiles,
// two in flight; lane (n, g) = (l % 32, l / 32) holds B[n][k0 + g*32 .. +32] and
// feeds 16-byte piece kk to MFMA step kk. A rows in LDS are 128 B, pieces
// XOR-swizzled by (row >> 1) & 7.
FG_DEVICE int a_swz32(int row, int piece) { return row * kBK + ((piece ^ ((row >> 1) & 7)) << 3); }

template <int CDT>
__global__ void __launch_bounds__(512) gemm_bf16_stream32_kernel(GemmArgs g, int epi) {
  constexpr int WAVES = 8, NT = 512, MB = 8, MROWS = 256;
  constexpr int AC = MROWS * (kBK / 8) / NT;  // 4
  __shared__ __attribute__((aligned(16))) uint16_t As[2][MROWS * kBK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g2 = lane >> 5;
  const int z = blockIdx.y;
  const int n_base = blockIdx.x * (WAVES * 32) + wave * 32;
  if (g.row_active && !tile_has_active_row(g, 0, g.M)) return;

  const uint16_t* Ab = (const uint16_t*)g.A + z * g.a_batch;
  const uint16_t* Bb = (const uint16_t*)g.B + z * g.b_batch;
  const v4u* dummy = (const v4u*)Bb;
  const int nb = min(n_base + (lane & 31), g.N - 1);
  const uint16_t* bsrc = Bb + (int64_t)nb * g.ldb + g2 * 32;
  const uint16_t* a_src = Ab + (tid & 7) * 8;
  int64_t a_off[AC];
  int a_dst[AC];
#pragma unroll
  for (int c = 0; c < AC; ++c) {
    int idx = tid + c * NT;
    int r = idx >> 3;
    int m = min(r, g.M - 1);
    int src_row = g.a_rows ? g.a_rows[m] : m;
    a_off[c] = (int64_t)src_row * g.lda;
    a_dst[c] = a_swz32(r, idx & 7);
  }
  floatx16 acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

  const int ktiles = g.K / kBK;  // even (host check)
  v4u w0[4], w1[4], a0[AC], a1[AC];
#define FG_ISSUE(W, A, KT)                                                                                  \
  {                                                                                                         \
    const int kt_ = (KT);                                                                                   \
    const bool live_ = kt_ < ktiles;                                                                        \
    _Pragma("unroll") for (int c = 0; c < AC; ++c) A[c] = live_ ? *(const v4u*)(a_src + a_off[c] + kt_ * kBK) : *dummy; \
    _Pragma("unroll") for (int q = 0; q < 4; ++q) W[q] = live_ ? *(const v4u*)(bsrc + kt_ * kBK + q * 8) : *dummy; \
  }
#define FG_STEP(W, A_NEXT, U)                                                                               \
  {                                                                                                         \
    const int cur = (kt0 + (U)) & 1;                                                                        \
    _Pragma("unroll") for (int kk = 0; kk < 4; ++kk) {                                                      \
      const bf16x8 wf = __builtin_bit_cast(bf16x8, W[kk]);                                                  \
      _Pragma("unroll") for (int i = 0; i < MB; ++i) {                                                      \
        const bf16x8 af = *(const bf16x8*)&As[cur][a_swz32(i * 32 + (lane & 31), g2 * 4 + kk)];             \
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, af, acc[i], 0, 0, 0);                          \
      }                                                                                                     \
    }                                                                                                       \
    _Pragma("unroll") for (int c = 0; c < AC; ++c) *(v4u*)&As[cur ^ 1][a_dst[c]] = A_NEXT[c];             \
  }
  FG_ISSUE(w0, a0, 0)
  FG_ISSUE(w1, a1, 1)
#pragma unroll
  for (int c = 0; c < AC; ++c) *(v4u*)&As[0][a_dst[c]] = a0[c];
  __syncthreads();
  for (int kt0 = 0; kt0 < ktiles; kt0 += 2) {
    FG_STEP(w0, a1, 0) FG_ISSUE(w0, a0, kt0 + 2) __syncthreads();
    FG_STEP(w1, a0, 1) FG_ISSUE(w1, a1, kt0 + 3) __syncthreads();
  }
#undef FG_ISSUE
#undef FG_STEP

  // Epilogue: acc[i] is the C^T tile (n rows, m columns) -> lane owns column m.
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    const int m = i * 32 + (lane & 31);
    if (m >= g.M) continue;
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const int n = n_base + v4 * 8 + g2 * 4;
      float o[4] = {acc[i][4 * v4], acc[i][4 * v4 + 1], acc[i][4 * v4 + 2], acc[i][4 * v4 + 3]};
      if (epi == kEpiNone && n + 3 < g.N && (g.ldc & 3) == 0) {
        if constexpr (CDT == fg::kBF16) {
          *(uint2*)((uint16_t*)g.C + z * g.c_batch + (int64_t)m * g.ldc + n) =
              make_uint2(fg::pack_bf16x2(o[0], o[1]), fg::pack_bf16x2(o[2], o[3]));
        } else {
          *(float4*)((float*)g.C + z * g.c_batch + (int64_t)m * g.ldc + n) = make_float4(o[0], o[1], o[2], o[3]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) epilogue_store<CDT, fg::kBF16>(g, z, m, n + e, o[e], epi);
      }
    }
  }
}

template <int MB, int WAVES, int PF>
void launch_stream(const GemmArgs& g, int out_dtype, int epi, int batch, hipStream_t s) {
  dim3 grid((g.N + WAVES * 16 - 1) / (WAVES * 16), batch);
  if (out_dtype == fg::kBF16)
    hipLaunchKernelGGL((gemm_bf16_stream_kernel<MB, WAVES, PF, fg::kBF16>), grid, dim3(WAVES * 64), 0, s, g, epi);
  else
    hipLaunchKernelGGL((gemm_bf16_stream_kernel<MB, WAVES, PF, fg::kF32>), grid, dim3(WAVES * 64), 0, s, g, epi);
}

// 16-row blocks of A: 1, 2, 4 or 8 (M <= 128; above that the 32x32 variant runs).
constexpr int stream_mb(int M) { return M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8; }
constexpr int stream_pf(int) { return 4; }  // k-tiles in flight

// Can a weight-streaming kernel run this product? (bf16, M <= 256; K a multiple
// of 4 * 128 up to 128 rows, of 2 * 64 above.)
bool stream_gemm_ok(const GemmArgs& g) {
  if (g.M <= 128) return g.K % (kST * 4) == 0;
  return g.M <= 256 && g.K % (kBK * 2) == 0;
}

// The most waves per workgroup (<= 8) that still give >= 2 workgroups per CU
// (256 CUs) over the whole product. A staging needs MB*16*16 >= waves*64, and
// with more than 64 rows of A fewer than 4 waves leave too many staging chunks
// per thread.
void launch_stream_gemm(const GemmArgs& g, int out_dtype, int epi, int batch, hipStream_t s) {
  if (g.M > 128) {
    dim3 grid((g.N + 255) / 256, batch);
    if (out_dtype == fg::kBF16)
      hipLaunchKernelGGL(gemm_bf16_stream32_kernel<fg::kBF16>, grid, dim3(512), 0, s, g, epi);
    else
      hipLaunchKernelGGL(gemm_bf16_stream32_kernel<fg::kF32>, grid, dim3(512), 0, s, g, epi);
    return;
  }
  const int mb = stream_mb(g.M);
  auto wgs = [&](int waves) { return (long)((g.N + waves * 16 - 1) / (waves * 16)) * batch; };
  const int min_waves = mb >= 8 ? 4 : 2;
  int waves = std::min(8, mb * 4);
  while (waves > min_waves && wgs(waves) < 512) waves /= 2;
#define FG_STREAM(MBv, Wv) \
  if (mb == MBv && waves == Wv) { launch_stream<MBv, Wv, stream_pf(MBv)>(g, out_dtype, epi, batch, s); return; }
  FG_STREAM(1, 2) FG_STREAM(1, 4)
  FG_STREAM(2, 2) FG_STREAM(2, 4) FG_STREAM(2, 8)
  FG_STREAM(4, 2) FG_STREAM(4, 4) FG_STREAM(4, 8)
  FG_STREAM(8, 4) FG_STREAM(8, 8)
#undef FG_STREAM
}

// ----------------------------------------------------------------- fp32 FMA
template <int CDT>
__global__ void __launch_bounds__(256) gemm_f32_kernel(GemmArgs g, int epi) {
  constexpr int T = 64, BKf = 16;
  __shared__ float As[BKf][T + 1];
  __shared__ float Bs[BKf][T + 1];
  const int z = blockIdx.z;
  const int m0 = blockIdx.y * T, n0 = blockIdx.x * T;
  if (g.row_active && !tile_has_active_row(g, m0, T)) return;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const float* Ab = (const float*)g.A + z * g.a_batch;
  const float* Bb = (const float*)g.B + z * g.b_batch;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < g.K; k0 += BKf) {
    for (int e = threadIdx.x; e < T * BKf; e += 256) {
      int r = e / BKf, kk = e % BKf;
      int m = m0 + r, n = n0 + r, k = k0 + kk;
      float av = 0.0f, bv = 0.0f;
      if (m < g.M && k < g.K) {
        int src = g.a_rows ? g.a_rows[m] : m;
        av = Ab[(int64_t)src * g.lda + k];
      }
      if (n < g.N && k < g.K) bv = Bb[(int64_t)n * g.ldb + k];
      As[kk][r] = av;
      Bs[kk][r] = bv;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BKf; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) epilogue_store<CDT, fg::kF32>(g, z, m0 + ty * 4 + i, n0 + tx * 4 + j, acc[i][j], epi);
}

// fp32 Medusa block, split over K: blockIdx.z = z * ksplit + p takes k in [p * kper, (p + 1) * kper)
// of batch z's product and writes the raw sums to parts[p][z][m][n] (64 x 64 tile, 4 x 4 outputs
// per thread, each thread loading one 16-byte run of 4 k values of A and of B per 16-deep k-step).
// medusa_f32_combine_kernel finishes the block. The unsplit kernel above runs a 96 x 4096 x 4096
// bootstrap (the chain path's head 0, fp32 master weights) as 128 workgroups walking all of K.
template <int DUMMY>
__global__ void __launch_bounds__(256) gemm_f32_split_kernel(GemmArgs g, int ksplit, int kper, float* parts) {
  constexpr int T = 64, BKf = 16;
  __shared__ float As[BKf][T + 1];
  __shared__ float Bs[BKf][T + 1];
  const int z = blockIdx.z / ksplit, sp = blockIdx.z % ksplit;
  const int m0 = blockIdx.y * T, n0 = blockIdx.x * T;
  const int k_begin = sp * kper, k_end = min(g.K, k_begin + kper);
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const float* Ab = (const float*)g.A + z * g.a_batch;
  const float* Bb = (const float*)g.B + z * g.b_batch;
  // loader: thread t takes row t / 4 and k run 4 * (t % 4) of the 64 x 16 tile of A and of B
  const int lr = threadIdx.x >> 2, lk = (threadIdx.x & 3) * 4;
  const bool a_ok = m0 + lr < g.M, b_ok = n0 + lr < g.N;
  const float* arow = Ab + (int64_t)(a_ok ? m0 + lr : 0) * g.lda;
  const float* brow = Bb + (int64_t)(b_ok ? n0 + lr : 0) * g.ldb;
  float acc[4][4] = {};
  for (int k0 = k_begin; k0 < k_end; k0 += BKf) {
    const int k = k0 + lk;
    float4 av = make_float4(0.0f, 0.0f, 0.0f, 0.0f), bv = av;
    if (k + 4 <= k_end) {
      if (a_ok) av = *(const float4*)(arow + k);
      if (b_ok) bv = *(const float4*)(brow + k);
    } else {  // the part's last k-step (K a multiple of 4 keeps runs whole)
      if (a_ok && k < k_end) av = *(const float4*)(arow + k);
      if (b_ok && k < k_end) bv = *(const float4*)(brow + k);
    }
    As[lk][lr] = av.x; As[lk + 1][lr] = av.y; As[lk + 2][lr] = av.z; As[lk + 3][lr] = av.w;
    Bs[lk][lr] = bv.x; Bs[lk + 1][lr] = bv.y; Bs[lk + 2][lr] = bv.z; Bs[lk + 3][lr] = bv.w;
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BKf; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  float* dst = parts + ((int64_t)sp * gridDim.z / ksplit + z) * (int64_t)g.M * g.N;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i, n = n0 + tx * 4;
    if (m < g.M && n < g.N)  // N % 4 == 0
      *(float4*)(dst + (int64_t)m * g.N + n) = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
  }
}

// out[z * M + m, n] = R[m, n] + SiLU(sum_p parts[p][z][m][n] + bias[z][n]) in fp32 (the module's fp32
// forward: no intermediate rounding), parts summed in order; 4 columns per thread.
template <int ODT>
__global__ void __launch_bounds__(256) medusa_f32_combine_kernel(const float* __restrict__ parts, int ksplit,
                                                                 int heads, int M, int N,
                                                                 const float* __restrict__ bias,
                                                                 const float* __restrict__ R, int64_t ldr,
                                                                 void* __restrict__ out) {
  const int nq = N >> 2;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)heads * M * nq) return;
  const int c = (int)(idx % nq) * 4;
  const int64_t hm = idx / nq;  // h * M + m
  const int h = (int)(hm / M), m = (int)(hm % M);
  const int64_t plane = (int64_t)heads * M * N;
  float4 sv = *(const float4*)(parts + hm * N + c);
  for (int p = 1; p < ksplit; ++p) {
    const float4 pv = *(const float4*)(parts + p * plane + hm * N + c);
    sv.x += pv.x; sv.y += pv.y; sv.z += pv.z; sv.w += pv.w;
  }
  const float4 bv = *(const float4*)(bias + (int64_t)h * N + c);
  const float4 rv = *(const float4*)(R + (int64_t)m * ldr + c);
  const float v[4] = {rv.x + fg::silu_f32(sv.x + bv.x), rv.y + fg::silu_f32(sv.y + bv.y),
                      rv.z + fg::silu_f32(sv.z + bv.z), rv.w + fg::silu_f32(sv.w + bv.w)};
  if constexpr (ODT == fg::kBF16)
    *(uint2*)((uint16_t*)out + hm * N + c) = make_uint2(fg::pack_bf16x2(v[0], v[1]), fg::pack_bf16x2(v[2], v[3]));
  else
    *(float4*)((float*)out + hm * N + c) = make_float4(v[0], v[1], v[2], v[3]);
}

struct F32Split {
  int ksplit, kper;
};
// Splits of K (each a multiple of 16, at most 8) that bring heads x 64 x 64 tiles to about two
// workgroups per CU; 1 when the tiles alone fill the chip.
F32Split f32_split(int M, int N, int K, int heads) {
  const int64_t tiles = (int64_t)heads * ((M + 63) / 64) * ((N + 63) / 64);
  int ks = tiles >= 512 ? 1 : (int)std::min<int64_t>(8, (512 + tiles - 1) / tiles);
  ks = std::max(1, std::min(ks, K / 64));
  const int kper = ((K + ks - 1) / ks + 15) / 16 * 16;
  return {(K + kper - 1) / kper, kper};
}

int launch_gemm(const GemmArgs& g, int dtype, int out_dtype, int epi, int batch, hipStream_t s) {
  FG_REQUIRE(g.M > 0 && g.N > 0 && g.K > 0 && batch > 0, "gemm: empty shape");
  if (dtype == fg::kBF16) {
    FG_REQUIRE(g.K % kBK == 0, "gemm: bf16 path needs K % 64 == 0");
    FG_REQUIRE(g.lda % 8 == 0 && g.ldb % 8 == 0 && ((uintptr_t)g.A & 15) == 0 && ((uintptr_t)g.B & 15) == 0,
               "gemm: bf16 operands need 16-byte aligned rows");
    const bool wide_ok = g.N >= 512 && g.ldc % 4 == 0 && ((uintptr_t)g.C & 15) == 0 && (g.c_batch % 4) == 0;
    GemmArgs head = g;
    head.M = std::min(g.M, 256);
    if (stream_gemm_ok(head) && g.M <= 4096) {
      // 256-row slices, each streaming B once (the skinny kernel beats the
      // square-tile one here even when the product is compute-bound).
      const int es = out_dtype == fg::kBF16 ? 2 : 4;
      for (int m0 = 0; m0 < g.M; m0 += 256) {
        GemmArgs gc = g;
        gc.M = std::min(256, g.M - m0);
        if (g.a_rows) gc.a_rows = g.a_rows + m0;
        else gc.A = (const uint16_t*)g.A + (int64_t)m0 * g.lda;
        if (g.row_active) gc.row_active = g.row_active + m0;
        gc.C = (char*)g.C + (int64_t)m0 * g.ldc * es;
        if (g.R) gc.R = (const char*)g.R + (int64_t)m0 * g.ldr * (g.r_dtype == fg::kBF16 ? 2 : 4);
        launch_stream_gemm(gc, out_dtype, epi, batch, s);
      }
    } else if (wide_ok) {
      // Pick the M tile that pads M least (larger tile on ties).
      const int cands[3] = {192, 128, 64};
      int BM = 256, best = 1 << 30;
      for (int c : cands) {
        int waste = (g.M + c - 1) / c * c - g.M;
        if (waste < best) {
          best = waste;
          BM = c;
        }
      }
      int tm = (g.M + BM - 1) / BM, tn = (g.N + 255) / 256;
      dim3 grid(tm * tn, 1, batch);
#define FG_WIDE(BMv)                                                                                          \
  if (out_dtype == fg::kBF16)                                                                                  \
    hipLaunchKernelGGL((gemm_bf16_wide_kernel<BMv, fg::kBF16>), grid, dim3(256), 0, s, g, epi, tm, tn);        \
  else                                                                                                         \
    hipLaunchKernelGGL((gemm_bf16_wide_kernel<BMv, fg::kF32>), grid, dim3(256), 0, s, g, epi, tm, tn);
      if (BM == 192) { FG_WIDE(192) }
      else if (BM == 128) { FG_WIDE(128) }
      else { FG_WIDE(64) }
#undef FG_WIDE
    } else if (g.M <= 64) {
      constexpr int BM = 64, BN = 128;
      int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
      dim3 grid(tm * tn, 1, batch);
      if (out_dtype == fg::kBF16)
        hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, 32, 64, fg::kBF16>), grid, dim3(256), 0, s, g, epi, tm, tn);
      else
        hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, 32, 64, fg::kF32>), grid, dim3(256), 0, s, g, epi, tm, tn);
    } else {
      constexpr int BM = 128, BN = 128;
      int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
      dim3 grid(tm * tn, 1, batch);
      if (out_dtype == fg::kBF16)
        hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, 64, 64, fg::kBF16>), grid, dim3(256), 0, s, g, epi, tm, tn);
      else
        hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, 64, 64, fg::kF32>), grid, dim3(256), 0, s, g, epi, tm, tn);
    }
  } else {
    dim3 grid((g.N + 63) / 64, (g.M + 63) / 64, batch);
    if (out_dtype == fg::kBF16)
      hipLaunchKernelGGL(gemm_f32_kernel<fg::kBF16>, grid, dim3(256), 0, s, g, epi);
    else
      hipLaunchKernelGGL(gemm_f32_kernel<fg::kF32>, grid, dim3(256), 0, s, g, epi);
  }
  return fg::check_launch("gemm");
}

// LayerNorm of each row of h, once per Medusa head (affine per head).
template <int HDT, int ODT>
__global__ void __launch_bounds__(256) medusa_ln_kernel(const void* __restrict__ h, int64_t ldh, int H, int heads,
                                                        int batch, const float* __restrict__ ln_w,
                                                        const float* __restrict__ ln_b, float eps,
                                                        void* __restrict__ out) {
  const int b = blockIdx.x;
  __shared__ float red[8];
  float s = 0.0f;
  for (int i = threadIdx.x; i < H; i += 256) s += fg::load_elem<HDT>(h, (int64_t)b * ldh + i);
  s = fg::wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  const float mean = (red[0] + red[1] + red[2] + red[3]) / (float)H;
  __syncthreads();
  float v = 0.0f;
  for (int i = threadIdx.x; i < H; i += 256) {
    float d = fg::load_elem<HDT>(h, (int64_t)b * ldh + i) - mean;
    v += d * d;
  }
  v = fg::wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[4 + (threadIdx.x >> 6)] = v;
  __syncthreads();
  const float rstd = rsqrtf((red[4] + red[5] + red[6] + red[7]) / (float)H + eps);
  for (int hd = 0; hd < heads; ++hd)
    for (int i = threadIdx.x; i < H; i += 256) {
      float x = (fg::load_elem<HDT>(h, (int64_t)b * ldh + i) - mean) * rstd;
      fg::store_elem<ODT>(out, ((int64_t)hd * batch + b) * H + i, x * ln_w[hd * H + i] + ln_b[hd * H + i]);
    }
}

// LayerNorm of the Medusa block with one workgroup per (row, head): the row is held in
// registers (16-byte loads, H a multiple of 8, at most 8192), its mean and variance reduced
// over the workgroup, and the head's affine output written with 16-byte stores.
template <int HDT, int ODT>
__global__ void __launch_bounds__(256) medusa_ln_vec_kernel(const void* __restrict__ h, int64_t ldh, int H, int batch,
                                                            const float* __restrict__ ln_w,
                                                            const float* __restrict__ ln_b, float eps,
                                                            void* __restrict__ out) {
  constexpr int KMAX = 4;
  const int b = blockIdx.x, hd = blockIdx.y, tid = threadIdx.x;
  const int nchunk = H >> 3;
  const void* row = (const char*)h + (int64_t)b * ldh * (HDT == fg::kBF16 ? 2 : 4);
  __shared__ float red[8];
  float x[KMAX][8];
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int c = tid + k * 256;
    if (c < nchunk) {
      fg::load8<HDT>(row, (int64_t)c * 8, x[k]);
#pragma unroll
      for (int j = 0; j < 8; ++j) s += x[k][j];
    }
  }
  s = fg::wave_sum(s);
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  const float mean = (red[0] + red[1] + red[2] + red[3]) / (float)H;
  float v = 0.0f;
#pragma unroll
  for (int k = 0; k < KMAX; ++k)
    if (tid + k * 256 < nchunk) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float d = x[k][j] - mean;
        v += d * d;
      }
    }
  v = fg::wave_sum(v);
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = v;
  __syncthreads();
  const float rstd = rsqrtf((red[4] + red[5] + red[6] + red[7]) / (float)H + eps);
  const float* w = ln_w + (int64_t)hd * H;
  const float* bb = ln_b + (int64_t)hd * H;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int c = tid + k * 256;
    if (c < nchunk) {
      float wv[8], bv[8], y[8];
      fg::load8<fg::kF32>(w, (int64_t)c * 8, wv);
      fg::load8<fg::kF32>(bb, (int64_t)c * 8, bv);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = (x[k][j] - mean) * rstd * wv[j] + bv[j];
      fg::store8<ODT>(out, ((int64_t)hd * batch + b) * H + (int64_t)c * 8, y);
    }
  }
}

}  // namespace

extern "C" {

int fg_lm_head(const void* x, int dtype, int M, int K, int64_t ldx, const int32_t* row_index,
               const int32_t* row_active, const void* w, int64_t ldw, int N, void* out, int out_dtype, int64_t ldo,
               void* stream) {
  FG_REQUIRE(x && w && out, "fg_lm_head: null pointer");
  FG_REQUIRE(dtype == fg::kF32 || dtype == fg::kBF16, "fg_lm_head: dtype");
  GemmArgs g{};
  g.A = x; g.lda = ldx; g.a_rows = row_index; g.row_active = row_active;
  g.B = w; g.ldb = ldw;
  g.C = out; g.ldc = ldo;
  g.M = M; g.N = N; g.K = K;
  return launch_gemm(g, dtype, out_dtype, kEpiNone, 1, (hipStream_t)stream);
}

// The normalised rows, then (bf16, weight-streamed fc) the fp32 partial sums 16-byte aligned.
static size_t medusa_ln_bytes(int batch, int hidden, int heads, int dtype) {
  return ((size_t)batch * hidden * heads * fg::elem_bytes(dtype) + 15) & ~(size_t)15;
}

// The fp32 block's split-K path: H a multiple of 4, 16-byte aligned rows.
static bool medusa_f32_split_ok(int H, int64_t ldh) { return H % 4 == 0 && ldh % 4 == 0; }

size_t fg_medusa_heads_workspace(int batch, int hidden, int heads, int dtype) {
  if (batch <= 0 || hidden <= 0 || heads <= 0) return 256;
  size_t parts = 0;
  if (dtype == fg::kBF16) {
    parts = fg::medusa_stream_parts_bytes(batch, hidden, heads);
  } else if (medusa_f32_split_ok(hidden, hidden)) {
    const F32Split sp = f32_split(batch, hidden, hidden, heads);
    parts = (size_t)sp.ksplit * heads * batch * hidden * 4;
  }
  return medusa_ln_bytes(batch, hidden, heads, dtype) + parts + 256;
}

// out[h*B + b, :] = hidden[b] + SiLU(fc_h(LayerNorm_h(hidden[b]))) for each head h.
int fg_medusa_heads(const void* hidden, int dtype, int batch, int H, int64_t ldh, int heads, const float* ln_w,
                    const float* ln_b, float ln_eps, const void* fc_w, const void* fc_b, void* out, int out_dtype,
                    void* workspace, size_t workspace_bytes, void* stream) {
  FG_REQUIRE(hidden && ln_w && ln_b && fc_w && fc_b && out && workspace, "fg_medusa_heads: null pointer");
  FG_REQUIRE(batch > 0 && H > 0 && heads > 0, "fg_medusa_heads: empty shape");
  FG_REQUIRE(dtype == fg::kF32 || dtype == fg::kBF16, "fg_medusa_heads: dtype");
  FG_REQUIRE(workspace_bytes >= fg_medusa_heads_workspace(batch, H, heads, dtype) - 256, "fg_medusa_heads: workspace");
  hipStream_t s = (hipStream_t)stream;
  const bool vec = H % 8 == 0 && H <= 8 * 256 * 4 && ldh % 8 == 0 && ((uintptr_t)hidden & 15) == 0 &&
                   ((uintptr_t)workspace & 15) == 0 && ((uintptr_t)ln_w & 15) == 0 && ((uintptr_t)ln_b & 15) == 0;
  if (vec && dtype == fg::kBF16)
    hipLaunchKernelGGL((medusa_ln_vec_kernel<fg::kBF16, fg::kBF16>), dim3(batch, heads), dim3(256), 0, s, hidden, ldh,
                       H, batch, ln_w, ln_b, ln_eps, workspace);
  else if (vec)
    hipLaunchKernelGGL((medusa_ln_vec_kernel<fg::kF32, fg::kF32>), dim3(batch, heads), dim3(256), 0, s, hidden, ldh,
                       H, batch, ln_w, ln_b, ln_eps, workspace);
  else if (dtype == fg::kBF16)
    hipLaunchKernelGGL((medusa_ln_kernel<fg::kBF16, fg::kBF16>), dim3(batch), dim3(256), 0, s, hidden, ldh, H, heads,
                       batch, ln_w, ln_b, ln_eps, workspace);
  else
    hipLaunchKernelGGL((medusa_ln_kernel<fg::kF32, fg::kF32>), dim3(batch), dim3(256), 0, s, hidden, ldh, H, heads,
                       batch, ln_w, ln_b, ln_eps, workspace);
  int rc = fg::check_launch("fg_medusa_heads(ln)");
  if (rc) return rc;
  if (vec && dtype == fg::kBF16 && fg::medusa_stream_ok(batch, H, heads) && ldh % 4 == 0 &&
      ((uintptr_t)out & 15) == 0 && ((uintptr_t)fc_w & 15) == 0 && ((uintptr_t)fc_b & 7) == 0) {
    float* parts = (float*)((char*)workspace + medusa_ln_bytes(batch, H, heads, dtype));
    return fg::medusa_stream(workspace, batch, H, heads, fc_w, fc_b, hidden, ldh, dtype, out, out_dtype, parts, s);
  }
  GemmArgs g{};
  g.A = workspace; g.lda = H; g.a_batch = (int64_t)batch * H;
  g.B = fc_w; g.ldb = H; g.b_batch = (int64_t)H * H;
  g.C = out; g.ldc = H; g.c_batch = (int64_t)batch * H;
  g.bias = fc_b; g.bias_batch = H;
  g.R = hidden; g.ldr = ldh; g.r_batch = 0; g.r_dtype = dtype;
  g.M = batch; g.N = H; g.K = H;
  if (dtype == fg::kF32 && medusa_f32_split_ok(H, ldh) && ((uintptr_t)fc_w & 15) == 0 && ((uintptr_t)fc_b & 15) == 0 &&
      ((uintptr_t)hidden & 15) == 0 && ((uintptr_t)out & (out_dtype == fg::kBF16 ? 7 : 15)) == 0) {
    // fp32 heads: K split into parts that fill the chip, then the fp32 combine
    const F32Split sp = f32_split(batch, H, H, heads);
    float* parts = (float*)((char*)workspace + medusa_ln_bytes(batch, H, heads, dtype));
    const dim3 grid((H + 63) / 64, (batch + 63) / 64, heads * sp.ksplit);
    hipLaunchKernelGGL(gemm_f32_split_kernel<0>, grid, dim3(256), 0, s, g, sp.ksplit, sp.kper, parts);
    rc = fg::check_launch("fg_medusa_heads(f32 split)");
    if (rc) return rc;
    const int64_t threads = (int64_t)heads * batch * (H / 4);
    const dim3 cgrid((unsigned)((threads + 255) / 256));
    if (out_dtype == fg::kBF16)
      hipLaunchKernelGGL(medusa_f32_combine_kernel<fg::kBF16>, cgrid, dim3(256), 0, s, parts, sp.ksplit, heads, batch,
                         H, (const float*)fc_b, (const float*)hidden, ldh, out);
    else
      hipLaunchKernelGGL(medusa_f32_combine_kernel<fg::kF32>, cgrid, dim3(256), 0, s, parts, sp.ksplit, heads, batch,
                         H, (const float*)fc_b, (const float*)hidden, ldh, out);
    return fg::check_launch("fg_medusa_heads(f32 combine)");
  }
  return launch_gemm(g, dtype, out_dtype, kEpiMedusa, heads, s);
}

}  // extern "C"
