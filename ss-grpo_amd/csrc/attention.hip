// Tree-verify attention over the cached prefix plus the candidate tree.
//
// Query node n of sequence b (all q heads of one KV head, GQA) attends to the
// committed prefix keys [0, seq_len[b]) and to tree keys seq_len[b] + m for
// every node m whose bit is set in the node's 64-bit ancestor-or-self mask.
// The mask is applied to the scores in registers; no [B, 1, N, P+N] float mask
// is built (replaces flashgrpo/decoding/tree_attention.py:6-67 feeding the HF
// decoder's eager/SDPA attention, flashgrpo/models/qwen_flashgrpo_wrapper.py:172-180).
//
// bf16 path, one workgroup of 8 waves per (sequence, kv head, 256-row query tile):
//  * the query tile is the G*N rows (n-major, G = q heads per kv head) of one
//    KV head, so every K/V tile loaded from HBM serves all of them;
//  * each wave owns 32 query rows; two waves share a SIMD, so one wave's MFMAs
//    overlap the other's softmax arithmetic; a wave whose rows are all past the
//    tile only stages K/V;
//  * S^T = K Q^T (keys on the M side) puts one query per lane: the online
//    softmax row max / sum are per-lane values plus one exchange with lane^32;
//  * O^T += V^T P^T: P^T is fed straight from the S^T accumulators (bf16) as the
//    B operand; V is transposed into LDS while staging (2 keys x 8 dims per
//    thread) so the A operand reads two 8-byte runs per lane in the key order
//    of the accumulators; 4-key groups of V^T row d are stored XOR-swizzled by
//    (d >> 3) & 15, which keeps the staging writes and the fragment reads free
//    of bank conflicts;
//  * K/V tiles are double-buffered in LDS and staged through two register
//    stages: the global loads of tile t+2 are issued before tile t is computed
//    (two tiles in flight per workgroup), one barrier per 64-key tile;
//  * the ancestor mask is evaluated only on tiles that reach the tree keys, and
//    the running max (and the O rescale) only moves when a lane's max grows by
//    more than 2^8, so after the first keys the rescale is almost never taken.
// fp32 path: one wave per query row, exact online softmax in fp32.
#include "fg_common.h"

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
};

constexpr int kD = 128;            // head dim of the MFMA path
constexpr int kKT = 64;            // keys per tile
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kRowsTile = kWaves * 32;
constexpr int kKPitch = kD + 8;    // bf16 elements per K row in LDS
constexpr int kVPitch = kKT + 8;   // bf16 elements per V^T row in LDS
constexpr float kRescaleSlack = 8.0f;  // log2 units
static_assert(kKT * kD / 8 == 2 * kThreads, "staging: two 16-byte K and V chunks per thread");

FG_DEVICE int c_row32(int i, int lane) { return (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3); }

// Keys key0 .. key0+63 of one row: key0 + j is allowed when it is a prefix key
// (j < sh, sh = seq_len - key0) or tree node j - sh with its bit set in tree_bits.
// Shift amounts are kept in [0, 63].
FG_DEVICE uint64_t tile_allowed_mask(int sh, uint64_t tree_bits) {
  const uint64_t prefix = sh <= 0 ? 0ull : sh >= 64 ? ~0ull : ((1ull << sh) - 1ull);
  const uint64_t tree = sh >= 64 ? 0ull : sh >= 0 ? (tree_bits << sh) : sh <= -64 ? 0ull : (tree_bits >> -sh);
  return prefix | tree;
}

__global__ void __launch_bounds__(kThreads) tree_attn_bf16_kernel(AttnArgs a, int m_tiles) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kKT * kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][kD * kVPitch];

  const int mt = blockIdx.x % m_tiles;
  const int hkv = (blockIdx.x / m_tiles) % a.Hkv;
  const int b = blockIdx.x / (m_tiles * a.Hkv);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5;
  const int G = a.Hq / a.Hkv;
  const int M = G * a.N;
  const int s0 = a.seq_len[b];
  const int total = s0 + a.N;
  const int last_key = min(total, a.capacity) - 1;
  const int cb = a.row_map ? a.row_map[b] : b;
  const uint16_t* kbase = (const uint16_t*)a.k + (int64_t)cb * a.cache_batch + (int64_t)hkv * a.cache_head;
  const uint16_t* vbase = (const uint16_t*)a.v + (int64_t)cb * a.cache_batch + (int64_t)hkv * a.cache_head;

  // This lane's query row (column of S^T).
  const int row0 = mt * kRowsTile + wave * 32;
  const bool computes = row0 < M;   // wave-uniform
  const int r = row0 + (lane & 31);
  const bool row_ok = r < M;
  const int qn = row_ok ? r / G : 0;
  const int qh = hkv * G + (row_ok ? r % G : 0);
  const uint64_t anc = row_ok ? a.anc[(int64_t)b * a.anc_stride + qn] : 1ull;
  const uint64_t tree_bits = a.N >= 64 ? anc : anc & ((1ull << a.N) - 1);  // allowed tree nodes

  // Q^T fragments: step s covers d = s*16 + g*8 .. +8.
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

  // Staging. K: chunk c of thread t is row t/16 + 32c, dims (t%16)*8..+8.
  // V: thread t holds keys 2*(t/16) and 2*(t/16)+1 of dims (t%16)*8..+8 and
  // writes each V^T row as one 4-byte key pair.
  const int st_col = (tid & 15) * 8;
  const int st_row = tid >> 4;
  // Two register stages (named 16-byte vectors, not arrays, so they stay in VGPRs):
  // the loads of tile t+2 are issued before tile t is computed, so every tile's
  // loads are in flight across two tile computations.
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  v4u ka0, ka1, va0, va1, kb0, kb1, vb0, vb1;
#define FG_LOAD(K0, K1, V0, V1, KEY0)                                                      \
  {                                                                                        \
    const int key0_ = (KEY0);                                                              \
    const uint16_t* kp_ = kbase + st_col;                                                  \
    const uint16_t* vp_ = vbase + st_col;                                                  \
    K0 = *(const v4u*)(kp_ + (int64_t)min(key0_ + st_row, last_key) * kD);                 \
    K1 = *(const v4u*)(kp_ + (int64_t)min(key0_ + st_row + 32, last_key) * kD);            \
    V0 = *(const v4u*)(vp_ + (int64_t)min(key0_ + 2 * st_row, last_key) * kD);             \
    V1 = *(const v4u*)(vp_ + (int64_t)min(key0_ + 2 * st_row + 1, last_key) * kD);         \
  }
  // V^T row d, key pair p (keys 2p, 2p+1) lives at word 2*((p >> 1) ^ ((d >> 3) & 15)) + (p & 1).
  const int vsw_word = 2 * ((st_row >> 1) ^ ((st_col >> 3) & 15)) + (st_row & 1);
#define FG_STORE(K0, K1, V0, V1, BUF)                                                      \
  {                                                                                        \
    uint16_t* kd_ = &Ks[BUF][st_row * kKPitch + st_col];                                   \
    *(v4u*)(kd_) = K0;                                                                     \
    *(v4u*)(kd_ + 32 * kKPitch) = K1;                                                      \
    uint32_t* vt_ = (uint32_t*)&Vt[BUF][st_col * kVPitch] + vsw_word;                      \
    _Pragma("unroll") for (int e2 = 0; e2 < 4; ++e2) {                                     \
      vt_[(2 * e2) * (kVPitch / 2)] = __builtin_amdgcn_perm(V1[e2], V0[e2], 0x05040100u);     \
      vt_[(2 * e2 + 1) * (kVPitch / 2)] = __builtin_amdgcn_perm(V1[e2], V0[e2], 0x07060302u); \
    }                                                                                      \
  }

  // An even number of tiles: a padding tile past the keys is fully masked (its
  // loads re-read the last key) and leaves O and l unchanged.
  const int ntiles = ((total + kKT - 1) / kKT + 1) & ~1;
  FG_LOAD(ka0, ka1, va0, va1, 0)
  FG_LOAD(kb0, kb1, vb0, vb1, kKT)
  FG_STORE(ka0, ka1, va0, va1, 0)
  __syncthreads();
  for (int t0 = 0; t0 < ntiles; t0 += 2)
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int buf = h;
    const int key0 = (t0 + h) * kKT;
    if (h == 0) FG_LOAD(ka0, ka1, va0, va1, key0 + 2 * kKT)
    else FG_LOAD(kb0, kb1, vb0, vb1, key0 + 2 * kKT)

    if (computes) {
      // S^T for two 32-key blocks.
      floatx16 st[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) st[kb][i] = 0.0f;
#pragma unroll
        for (int s = 0; s < kD / 16; ++s) {
          bf16x8 kf = *(const bf16x8*)&Ks[buf][(kb * 32 + (lane & 31)) * kKPitch + s * 16 + g * 8];
          st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], st[kb], 0, 0, 0);
        }
      }
      if (key0 + kKT > s0) {  // tile reaches the tree keys (or the end)
        // Allowed keys of this tile as a 64-bit mask (bit j = key key0 + j), shifted
        // to this half-wave's first key; element i sits at bit kb*32 + c_row32(i, 0).
        const uint64_t allowed = tile_allowed_mask(s0 - key0, tree_bits) >> (g * 4);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const bool ok = (allowed >> (kb * 32 + c_row32(i, 0))) & 1ull;
            st[kb][i] = ok ? st[kb][i] : -INFINITY;
          }
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, st[kb][i]);
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      // Lazy rescale: the reference max only moves when some lane's max grew by
      // more than 2^kRescaleSlack, so p <= 2^kRescaleSlack and O / l is unchanged.
      const float m_new = fmaxf(m_run, tmax * sl2);
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
      float psum = 0.0f;
      bf16x8 pf[2][2];  // [kb][ks] B operand of P^T
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          uint32_t packed[4];
#pragma unroll
          for (int j = 0; j < 8; j += 2) {
            float p0 = __builtin_amdgcn_exp2f(fmaf(st[kb][ks * 8 + j], sl2, -m_sub));
            float p1 = __builtin_amdgcn_exp2f(fmaf(st[kb][ks * 8 + j + 1], sl2, -m_sub));
            psum += p0 + p1;
            packed[j / 2] = fg::pack_bf16x2(p0, p1);
          }
          pf[kb][ks] = __builtin_bit_cast(bf16x8, make_uint4(packed[0], packed[1], packed[2], packed[3]));
        }
      l_run += psum;
      // O^T += V^T P^T. Slot j of lane (g) holds key kb*32 + ks*16 + (j/4)*8 + g*4 + j%4.
#pragma unroll
      for (int db = 0; db < kD / 32; ++db) {
        const int dv = db * 32 + (lane & 31);
        const uint16_t* vrow = &Vt[buf][dv * kVPitch];
        const int sw = (dv >> 3) & 15;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            int kg = kb * 8 + ks * 4 + g;  // 4-key group of slots 0..3; slots 4..7 are group kg + 2
            uint2 lo = *(const uint2*)(vrow + 4 * (kg ^ sw));
            uint2 hi = *(const uint2*)(vrow + 4 * ((kg + 2) ^ sw));
            bf16x8 vf = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
            o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[kb][ks], o[db], 0, 0, 0);
          }
      }
    }
    if (h == 0) FG_STORE(kb0, kb1, vb0, vb1, 1)
    else FG_STORE(ka0, ka1, va0, va1, 0)
    __syncthreads();
  }
#undef FG_LOAD
#undef FG_STORE

  // Combine the two half-lanes' sums and write.
  float l = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  if (row_ok) {
    uint16_t* orow = (uint16_t*)a.out + (((int64_t)b * a.N + qn) * a.Hq + qh) * kD;
#pragma unroll
    for (int db = 0; db < kD / 32; ++db)
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        int d0 = db * 32 + c_row32(i, lane);
        uint32_t w0 = fg::pack_bf16x2(o[db][i] * inv, o[db][i + 1] * inv);
        uint32_t w1 = fg::pack_bf16x2(o[db][i + 2] * inv, o[db][i + 3] * inv);
        *(uint2*)(orow + d0) = make_uint2(w0, w1);
      }
  }
}

// fp32: one wave per (sequence, node, q head); lane owns head dims lane, lane+64.
__global__ void __launch_bounds__(64) tree_attn_f32_kernel(AttnArgs a) {
  const int qh = blockIdx.x % a.Hq;
  const int n = (blockIdx.x / a.Hq) % a.N;
  const int b = blockIdx.x / (a.Hq * a.N);
  const int lane = threadIdx.x;
  const int G = a.Hq / a.Hkv, hkv = qh / G;
  const int s0 = a.seq_len[b];
  const int cb = a.row_map ? a.row_map[b] : b;
  const float* kbase = (const float*)a.k + (int64_t)cb * a.cache_batch + (int64_t)hkv * a.cache_head;
  const float* vbase = (const float*)a.v + (int64_t)cb * a.cache_batch + (int64_t)hkv * a.cache_head;
  const float* qrow = (const float*)a.q + (((int64_t)b * a.N + n) * a.Hq + qh) * a.d;
  const uint64_t anc = a.anc[(int64_t)b * a.anc_stride + n];
  float q0 = lane < a.d ? qrow[lane] : 0.0f;
  float q1 = lane + 64 < a.d ? qrow[lane + 64] : 0.0f;
  float m = -INFINITY, l = 0.0f, o0 = 0.0f, o1 = 0.0f;
  const int total = s0 + a.N;
  for (int key = 0; key < total; ++key) {
    if (key >= s0) {
      int mm = key - s0;
      if (!((anc >> mm) & 1ull)) continue;
    }
    const float* kr = kbase + (int64_t)key * a.d;
    float part = (lane < a.d ? q0 * kr[lane] : 0.0f) + (lane + 64 < a.d ? q1 * kr[lane + 64] : 0.0f);
    float s = fg::wave_sum(part) * a.scale;
    float m_new = fmaxf(m, s);
    float alpha = expf(m - m_new);
    float p = expf(s - m_new);
    const float* vr = vbase + (int64_t)key * a.d;
    l = l * alpha + p;
    o0 = o0 * alpha + (lane < a.d ? p * vr[lane] : 0.0f);
    o1 = o1 * alpha + (lane + 64 < a.d ? p * vr[lane + 64] : 0.0f);
    m = m_new;
  }
  float* orow = (float*)a.out + (((int64_t)b * a.N + n) * a.Hq + qh) * a.d;
  if (lane < a.d) orow[lane] = o0 / l;
  if (lane + 64 < a.d) orow[lane + 64] = o1 / l;
}

}  // namespace

extern "C" int fg_tree_attention(const void* q, void* out, const void* k_cache, const void* v_cache, int dtype,
                                 int batch, int num_nodes, int q_heads, int kv_heads, int head_dim,
                                 int64_t cache_batch_stride, int64_t cache_head_stride, int capacity,
                                 const int32_t* seq_len, const int32_t* row_map, const uint64_t* anc,
                                 int64_t anc_batch_stride, float scale, void* stream) {
  FG_REQUIRE(q && out && k_cache && v_cache && seq_len && anc, "fg_tree_attention: null pointer");
  FG_REQUIRE(batch > 0 && num_nodes > 0 && num_nodes <= 64, "fg_tree_attention: num_nodes must be in [1, 64]");
  FG_REQUIRE(q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0, "fg_tree_attention: heads");
  FG_REQUIRE(capacity >= num_nodes, "fg_tree_attention: capacity");
  AttnArgs a;
  a.q = q; a.out = out; a.k = k_cache; a.v = v_cache;
  a.cache_batch = cache_batch_stride; a.cache_head = cache_head_stride; a.capacity = capacity;
  a.seq_len = seq_len; a.row_map = row_map; a.anc = anc; a.anc_stride = anc_batch_stride;
  a.N = num_nodes; a.Hq = q_heads; a.Hkv = kv_heads; a.d = head_dim; a.scale = scale;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == fg::kBF16) {
    FG_REQUIRE(head_dim == kD, "fg_tree_attention: bf16 path supports head_dim 128");
    FG_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)k_cache & 15) == 0 && ((uintptr_t)v_cache & 15) == 0 &&
                   cache_head_stride % 8 == 0 && cache_batch_stride % 8 == 0,
               "fg_tree_attention: 16-byte alignment");
    int M = (q_heads / kv_heads) * num_nodes;
    int m_tiles = (M + kRowsTile - 1) / kRowsTile;
    hipLaunchKernelGGL(tree_attn_bf16_kernel, dim3(batch * kv_heads * m_tiles), dim3(kThreads), 0, s, a, m_tiles);
  } else if (dtype == fg::kF32) {
    FG_REQUIRE(head_dim <= 128, "fg_tree_attention: fp32 path supports head_dim <= 128");
    hipLaunchKernelGGL(tree_attn_f32_kernel, dim3(batch * num_nodes * q_heads), dim3(64), 0, s, a);
  } else {
    return fg::fail("fg_tree_attention: dtype");
  }
  return fg::check_launch("fg_tree_attention");
}
