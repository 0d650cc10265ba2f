// The HF rolling engine's current-chunk attention (hla/latent/batched_engine.py:156-162) with its backward: per head,
// one softmax of the chunk's RoPE'd queries over its RoPE'd keys, q, k, v [B, 16, n, 128] bf16 (any strides, unit
// last), visibility from valid [B, n]: a valid query i sees the valid keys j <= i, an invalid query sees every key of
// the chunk (its row stays finite; the engine never reads it). Outputs o [B, 16, n, 128] fp32 and lse [B, 16, n] fp32
// (natural log); the engine merges them with the latent history blocks by LSE.
//
// All three kernels run one wave per (batch row, head, 16-row block) on v_mfma_f32_16x16x32_bf16 for the score
// blocks (both operands rows of 128 dims, 16 bytes per lane) and v_mfma_f32_16x16x16_bf16 for the products over
// keys or queries, whose transposed operand comes from a wave-private LDS copy of the tile read by
// ds_read_b64_tr_b16:
//   * chunk_fwd: S^T = K Q^T per 16-key tile, online softmax per query column, O^T += V^T P^T;
//   * chunk_dq: delta = dO . O per query first (written for chunk_dkdv), then per key tile S^T and dP^T = V dO^T,
//     dS^T = P^T (dP^T - delta + dlse) scale, dQ^T += K^T dS^T;
//   * chunk_dkdv: per query tile S = Q K^T and dP = dO V^T against the block's K^T / V^T in registers, then
//     dV^T += dO^T P and dK^T += Q^T dS.
// P and dS are rounded to bf16 as MFMA operands (fp32 accumulation); dO is rounded to bf16 for the products.
// Each kernel loads its next tile (rows, row constants and valid bytes) while it computes the current one.
#include "common.h"

namespace hla {
namespace {

constexpr int kD = 128;              // head dim
constexpr int kHF = 16;              // heads
constexpr int kTS = kD + 16;         // LDS row stride of a tile, bf16 (conflict-free transposed reads)

struct HfChunkParams {
  const uint16_t *q, *k, *v;
  int64_t q_sb, q_sh, q_si, k_sb, k_sh, k_si, v_sb, v_sh, v_si;
  const uint8_t* valid;  // [B, n] (nonzero = valid)
  int64_t valid_sb;
  int n;
  float scale, scale_log2;
  float* o;  // fp32
  int64_t o_sb, o_sh, o_si;
  float* lse;  // [B, 16, n] natural log
  int64_t l_sb, l_sh;
  // backward
  const float* dout;  // fp32, strides of o
  int64_t d_sb, d_sh, d_si;
  const float* dlse;  // [B, 16, n] (lse strides) or null
  float* delta;       // [B, 16, n] (lse strides), written by chunk_dq
  float *dq, *dk, *dv;  // fp32 [B, 16, n, 128]
  int64_t g_sb, g_sh, g_si;
};

__device__ __forceinline__ bool visible(const uint8_t* vrow, int n, int i, int j) {
  if (i >= n || j >= n) return false;
  return vrow[i] ? (vrow[j] != 0 && j <= i) : true;
}

// 8 fp32 of a row -> 8 bf16 (round to nearest even), the 16-byte operand piece
__device__ __forceinline__ u32x4 f32x8_to_bf16(const float* p) {
  const floatx4 a = *reinterpret_cast<const floatx4*>(p), b = *reinterpret_cast<const floatx4*>(p + 4);
  return u32x4{pack2(a[0], a[1]), pack2(a[2], a[3]), pack2(b[0], b[1]), pack2(b[2], b[3])};
}

// A operand of a product over the tile's 16 rows for output rows [16nt, 16nt + 16) of the transposed tile: lane
// (g, hq) receives tile[4g + e][16nt + hq], e < 4 (the transposing read takes row 4g + hq / 4, columns
// 16nt + 4 (hq % 4) .. + 3 in each 16-lane group)
__device__ __forceinline__ short4v tile_t(const uint16_t* ts, int nt, int g, int hq) {
  const uint16_t* p = ts + (4 * g + (hq >> 2)) * kTS + 16 * nt + 4 * (hq & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)p);
}

__device__ __forceinline__ short4v pack4(const float (&x)[4]) {
  const uint32_t p01 = pack2_hw(x[0], x[1]), p23 = pack2_hw(x[2], x[3]);
  return short4v{(short)(p01 & 0xffffu), (short)(p01 >> 16), (short)(p23 & 0xffffu), (short)(p23 >> 16)};
}

// Keys the queries [q0, q0 + 16) may see: up to the block's last query, or the whole chunk when one of them is
// invalid (wave-uniform).
__device__ __forceinline__ int key_end(const uint8_t* vrow, int n, int q0, int hq) {
  const int qi = q0 + hq;
  const bool invalid_q = qi < n && vrow[qi] == 0;
  return __any(invalid_q) ? n : min(n, q0 + 16);
}

__global__ __launch_bounds__(64) void chunk_fwd(HfChunkParams a) {
  __shared__ __attribute__((aligned(16))) uint16_t vs[16 * kTS];
  const int lane = threadIdx.x, hq = lane & 15, g = lane >> 4;
  const int q0 = blockIdx.x * 16, h = blockIdx.y, b = blockIdx.z;
  const uint8_t* vrow = a.valid + (int64_t)b * a.valid_sb;
  const uint16_t* qh = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  const uint16_t* kh = a.k + (int64_t)b * a.k_sb + (int64_t)h * a.k_sh;
  const uint16_t* vh = a.v + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh;
  const int qi = q0 + hq;                 // this lane's query column
  const int qr = min(qi, a.n - 1);
  u32x4 qb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) qb[i] = ld16(qh + (int64_t)qr * a.q_si + 32 * i + 8 * g);
  floatx4 oacc[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) oacc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const int kend = key_end(vrow, a.n, q0, hq);
  const bool q_valid = qi < a.n && vrow[qr] != 0;
  // tile k0's K rows (A operand: key k0 + hq), V rows k0 .. k0 + 15 (piece c = it * 64 + lane is row c / 16,
  // 16 c % 16) and the valid bytes of keys k0 + 4g + r; the next tile's are loaded while a tile is computed
  auto load_tile = [&](int k0, u32x4 (&kA)[4], u32x4 (&vr)[4], uint8_t (&kv)[4]) {
    const int key = min(k0 + hq, a.n - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) kA[i] = ld16(kh + (int64_t)key * a.k_si + 32 * i + 8 * g);
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int c = it * 64 + lane, row = min(k0 + (c >> 4), a.n - 1);
      vr[it] = ld16(vh + (int64_t)row * a.v_si + (c & 15) * 8);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) kv[r] = vrow[min(k0 + 4 * g + r, a.n - 1)];
  };
  u32x4 kA[4], vr[4];
  uint8_t kv[4];
  if (kend > 0) load_tile(0, kA, vr, kv);
  for (int k0 = 0; k0 < kend; k0 += 16) {
    u32x4 kN[4], vN[4];
    uint8_t kvN[4];
    if (k0 + 16 < kend) load_tile(k0 + 16, kN, vN, kvN);
    floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) s = mfma16x16x32(kA[i], qb[i], s);
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int c = it * 64 + lane;
      st16(vs + (c >> 4) * kTS + (c & 15) * 8, vr[it]);
    }
    float sc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // visible(): a valid query sees the valid keys up to itself, an invalid one all
      const int j = k0 + 4 * g + r;
      const bool vis = qi < a.n && j < a.n && (q_valid ? (kv[r] != 0 && j <= qi) : true);
      sc[r] = vis ? s[r] * a.scale_log2 : -INFINITY;
    }
    const float mx = wave_max16x4_nn(max_nn(max_nn(sc[0], sc[1]), max_nn(sc[2], sc[3])));
    const bool raise = mx > m + 8.f;  // lazy rescale (the exponentials stay below 2^8)
    if (__any(raise)) {
      const float m_new = raise ? mx : m;
      // 0 on the first raise (m = -inf); 1 in a column that does not raise, which may still have no visible key
      // (a valid query after left padding, beside padding queries that see every key)
      const float alpha = raise ? fast_exp2(m - m_new) : 1.f;
      l *= alpha;
      m = m_new;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) oacc[nt] = oacc[nt] * alpha;
    }
    const float m_use = m == -INFINITY ? 0.f : m;
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = fast_exp2(sc[r] - m_use);
    l += (p[0] + p[1]) + (p[2] + p[3]);
    const short4v pb = pack4(p);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) oacc[nt] = mfma16x16x16(tile_t(vs, nt, g, hq), pb, oacc[nt]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kA[i] = kN[i];
      vr[i] = vN[i];
      kv[i] = kvN[i];
    }
  }
  l = wave_sum16x4(l);
  if (qi < a.n) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    float* op = a.o + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)qi * a.o_si + 4 * g;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) *reinterpret_cast<floatx4*>(op + 16 * nt) = oacc[nt] * inv;
    if (g == 0)
      a.lse[(int64_t)b * a.l_sb + (int64_t)h * a.l_sh + qi] = l > 0.f ? (m + log2f(l)) * kLn2 : -INFINITY;
  }
}

__global__ __launch_bounds__(64) void chunk_dq(HfChunkParams a) {
  __shared__ __attribute__((aligned(16))) uint16_t ks[16 * kTS];
  const int lane = threadIdx.x, hq = lane & 15, g = lane >> 4;
  const int q0 = blockIdx.x * 16, h = blockIdx.y, b = blockIdx.z;
  const uint8_t* vrow = a.valid + (int64_t)b * a.valid_sb;
  const uint16_t* qh = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  const uint16_t* kh = a.k + (int64_t)b * a.k_sb + (int64_t)h * a.k_sh;
  const uint16_t* vh = a.v + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh;
  const int qi = q0 + hq, qr = min(qi, a.n - 1);
  const int64_t lrow = (int64_t)b * a.l_sb + (int64_t)h * a.l_sh;
  u32x4 qb[4], db[4];
  float dsum = 0.f;
  {
    const float* dp = a.dout + (int64_t)b * a.d_sb + (int64_t)h * a.d_sh + (int64_t)qr * a.d_si;
    const float* op = a.o + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)qr * a.o_si;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qb[i] = ld16(qh + (int64_t)qr * a.q_si + 32 * i + 8 * g);
      db[i] = f32x8_to_bf16(dp + 32 * i + 8 * g);
      const floatx4 d0 = *reinterpret_cast<const floatx4*>(dp + 32 * i + 8 * g);
      const floatx4 d1 = *reinterpret_cast<const floatx4*>(dp + 32 * i + 8 * g + 4);
      const floatx4 o0 = *reinterpret_cast<const floatx4*>(op + 32 * i + 8 * g);
      const floatx4 o1 = *reinterpret_cast<const floatx4*>(op + 32 * i + 8 * g + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) dsum += d0[e] * o0[e] + d1[e] * o1[e];
    }
  }
  // delta = dO . O of the lane's query (the four lanes of the column hold a quarter of the dims each)
  dsum += __shfl_xor(dsum, 16);
  dsum += __shfl_xor(dsum, 32);
  const float delta = dsum;
  if (g == 0 && qi < a.n) a.delta[lrow + qi] = delta;
  const float lse2 = qi < a.n ? a.lse[lrow + qi] * kLog2e : 0.f;
  const float dl = a.dlse && qi < a.n ? a.dlse[lrow + qi] : 0.f;
  floatx4 acc[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) acc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int kend = key_end(vrow, a.n, q0, hq);
  const bool q_valid = qi < a.n && vrow[qr] != 0;
  // tile k0's K and V rows (A operands: key k0 + hq) and the valid bytes of keys k0 + 4g + r; the next tile's are
  // loaded while a tile is computed
  auto load_tile = [&](int k0, u32x4 (&kA)[4], u32x4 (&vA)[4], uint8_t (&kv)[4]) {
    const int key = min(k0 + hq, a.n - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kA[i] = ld16(kh + (int64_t)key * a.k_si + 32 * i + 8 * g);
      vA[i] = ld16(vh + (int64_t)key * a.v_si + 32 * i + 8 * g);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) kv[r] = vrow[min(k0 + 4 * g + r, a.n - 1)];
  };
  u32x4 kA[4], vA[4];
  uint8_t kv[4];
  if (kend > 0) load_tile(0, kA, vA, kv);
  for (int k0 = 0; k0 < kend; k0 += 16) {
    u32x4 kN[4], vN[4];
    uint8_t kvN[4];
    if (k0 + 16 < kend) load_tile(k0 + 16, kN, vN, kvN);
    floatx4 s = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s = mfma16x16x32(kA[i], qb[i], s);
      dp = mfma16x16x32(vA[i], db[i], dp);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) st16(ks + hq * kTS + 32 * i + 8 * g, kA[i]);  // K tile rows k0 + hq (row-major)
    float ds[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // visible(): a valid query sees the valid keys up to itself, an invalid one all
      const int j = k0 + 4 * g + r;
      const bool vis = qi < a.n && j < a.n && (q_valid ? (kv[r] != 0 && j <= qi) : true);
      const float p = vis ? fast_exp2(s[r] * a.scale_log2 - lse2) : 0.f;
      ds[r] = p * (dp[r] - delta + dl) * a.scale;
    }
    const short4v dsb = pack4(ds);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) acc[nt] = mfma16x16x16(tile_t(ks, nt, g, hq), dsb, acc[nt]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kA[i] = kN[i];
      vA[i] = vN[i];
      kv[i] = kvN[i];
    }
  }
  if (qi < a.n) {
    float* gp = a.dq + (int64_t)b * a.g_sb + (int64_t)h * a.g_sh + (int64_t)qi * a.g_si + 4 * g;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) *reinterpret_cast<floatx4*>(gp + 16 * nt) = acc[nt];
  }
}

__global__ __launch_bounds__(64) void chunk_dkdv(HfChunkParams a) {
  __shared__ __attribute__((aligned(16))) uint16_t qs[16 * kTS];
  __shared__ __attribute__((aligned(16))) uint16_t dos[16 * kTS];
  const int lane = threadIdx.x, hq = lane & 15, g = lane >> 4;
  const int j0 = blockIdx.x * 16, h = blockIdx.y, b = blockIdx.z;
  const uint8_t* vrow = a.valid + (int64_t)b * a.valid_sb;
  const uint16_t* qh = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  const uint16_t* kh = a.k + (int64_t)b * a.k_sb + (int64_t)h * a.k_sh;
  const uint16_t* vh = a.v + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh;
  const float* dh = a.dout + (int64_t)b * a.d_sb + (int64_t)h * a.d_sh;
  const int64_t lrow = (int64_t)b * a.l_sb + (int64_t)h * a.l_sh;
  const int kj = j0 + hq, kr = min(kj, a.n - 1);  // this lane's key column
  u32x4 kb[4], vb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kb[i] = ld16(kh + (int64_t)kr * a.k_si + 32 * i + 8 * g);
    vb[i] = ld16(vh + (int64_t)kr * a.v_si + 32 * i + 8 * g);
  }
  floatx4 dka[8], dva[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) dka[nt] = dva[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
  const bool k_valid = kj < a.n && vrow[kr] != 0;
  // the first query tile at or after q0 that contributes: a block of queries before the keys does so only through
  // its invalid queries (which see every key)
  auto next_tile = [&](int q0) {
    while (q0 < a.n && q0 + 15 < j0 && !__any(q0 + hq < a.n && vrow[q0 + hq] == 0)) q0 += 16;
    return q0;
  };
  // query tile q0's Q rows and dO rows (bf16, A operands: query q0 + hq), the row constants and valid bytes of the
  // four queries 4g + r of this lane's part of S; the next contributing tile's are loaded while a tile is computed
  struct QTile {
    u32x4 qA[4], dA[4];
    float lse2[4], del[4], dl[4];
    uint8_t qv[4];
  };
  auto load_tile = [&](int q0, QTile& t) {
    const int qr = min(q0 + hq, a.n - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      t.qA[i] = ld16(qh + (int64_t)qr * a.q_si + 32 * i + 8 * g);
      t.dA[i] = f32x8_to_bf16(dh + (int64_t)qr * a.d_si + 32 * i + 8 * g);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int q = min(q0 + 4 * g + r, a.n - 1);
      t.lse2[r] = a.lse[lrow + q] * kLog2e;
      t.del[r] = a.delta[lrow + q];
      t.dl[r] = a.dlse ? a.dlse[lrow + q] : 0.f;
      t.qv[r] = vrow[q];
    }
  };
  QTile cur;
  int q0 = next_tile(0);
  if (q0 < a.n) load_tile(q0, cur);
  while (q0 < a.n) {
    const int q1 = next_tile(q0 + 16);
    QTile nxt;
    if (q1 < a.n) load_tile(q1, nxt);
    const u32x4 (&qA)[4] = cur.qA;
    const u32x4 (&dA)[4] = cur.dA;
    const float (&lse2)[4] = cur.lse2;
    const float (&del)[4] = cur.del;
    const float (&dl)[4] = cur.dl;
    floatx4 s = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s = mfma16x16x32(qA[i], kb[i], s);   // S[q0 + 4g + r][kj]
      dp = mfma16x16x32(dA[i], vb[i], dp);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      st16(qs + hq * kTS + 32 * i + 8 * g, qA[i]);
      st16(dos + hq * kTS + 32 * i + 8 * g, dA[i]);
    }
    float p[4], ds[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // visible(): a valid query sees the valid keys up to itself, an invalid one all
      const int qq = q0 + 4 * g + r;
      const bool vis = qq < a.n && kj < a.n && (cur.qv[r] != 0 ? (k_valid && kj <= qq) : true);
      p[r] = vis ? fast_exp2(s[r] * a.scale_log2 - lse2[r]) : 0.f;
      ds[r] = p[r] * (dp[r] - del[r] + dl[r]) * a.scale;
    }
    const short4v pb = pack4(p), dsb = pack4(ds);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      dva[nt] = mfma16x16x16(tile_t(dos, nt, g, hq), pb, dva[nt]);
      dka[nt] = mfma16x16x16(tile_t(qs, nt, g, hq), dsb, dka[nt]);
    }
    cur = nxt;
    q0 = q1;
  }
  if (kj < a.n) {
    float* kp = a.dk + (int64_t)b * a.g_sb + (int64_t)h * a.g_sh + (int64_t)kj * a.g_si + 4 * g;
    float* vp = a.dv + (int64_t)b * a.g_sb + (int64_t)h * a.g_sh + (int64_t)kj * a.g_si + 4 * g;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      *reinterpret_cast<floatx4*>(kp + 16 * nt) = dka[nt];
      *reinterpret_cast<floatx4*>(vp + 16 * nt) = dva[nt];
    }
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_operands(const HfChunkParams& p, int B, int heads, int head_dim, const char* what) {
  HLA_REQUIRE(B >= 0 && p.n >= 0, HLA_S6_EINVAL, "%s: negative sizes", what);
  HLA_REQUIRE(heads == kHF && head_dim == kD, HLA_S6_EUNSUPPORTED, "%s: %d heads x %d dims (the kernels take 16 x 128)",
              what, heads, head_dim);
  HLA_REQUIRE(p.q && p.k && p.v && p.valid && p.lse, HLA_S6_EINVAL, "%s: null pointer argument", what);
  HLA_REQUIRE(aligned16(p.q) && aligned16(p.k) && aligned16(p.v) && p.q_sb % 8 == 0 && p.q_sh % 8 == 0 &&
                  p.q_si % 8 == 0 && p.k_sb % 8 == 0 && p.k_sh % 8 == 0 && p.k_si % 8 == 0 && p.v_sb % 8 == 0 &&
                  p.v_sh % 8 == 0 && p.v_si % 8 == 0,
              HLA_S6_EINVAL, "%s: q / k / v rows must be 16-byte aligned (strides multiples of 8)", what);
  HLA_REQUIRE(aligned16(p.o) && p.o_sb % 4 == 0 && p.o_sh % 4 == 0 && p.o_si % 4 == 0, HLA_S6_EINVAL,
              "%s: o rows must be 16-byte aligned (strides multiples of 4)", what);
  return HLA_S6_OK;
}

}  // namespace
}  // namespace hla

extern "C" int hla_s6_hf_chunk_forward(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_si, const void* k,
                                       int64_t k_sb, int64_t k_sh, int64_t k_si, const void* v, int64_t v_sb,
                                       int64_t v_sh, int64_t v_si, const uint8_t* valid, int64_t valid_sb,
                                       int32_t B, int32_t heads, int32_t n, int32_t head_dim, float scale, float* o,
                                       int64_t o_sb, int64_t o_sh, int64_t o_si, float* lse, int64_t l_sb,
                                       int64_t l_sh, void* stream) {
  using namespace hla;
  HfChunkParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.q_sb = q_sb, p.q_sh = q_sh, p.q_si = q_si, p.k_sb = k_sb, p.k_sh = k_sh, p.k_si = k_si;
  p.v_sb = v_sb, p.v_sh = v_sh, p.v_si = v_si;
  p.valid = valid;
  p.valid_sb = valid_sb;
  p.n = n;
  p.scale = scale;
  p.scale_log2 = scale * kLog2e;
  p.o = o, p.o_sb = o_sb, p.o_sh = o_sh, p.o_si = o_si;
  p.lse = lse, p.l_sb = l_sb, p.l_sh = l_sh;
  if (B == 0 || n == 0) return HLA_S6_OK;
  int rc = check_operands(p, B, heads, head_dim, "hf_chunk_forward");
  if (rc != HLA_S6_OK) return rc;
  HLA_REQUIRE(o != nullptr, HLA_S6_EINVAL, "hf_chunk_forward: null output");
  hipLaunchKernelGGL(chunk_fwd, dim3((unsigned)((n + 15) / 16), kHF, (unsigned)B), dim3(64), 0, as_stream(stream), p);
  return check_launch("hf_chunk_forward");
}

extern "C" int hla_s6_hf_chunk_backward(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_si, const void* k,
                                        int64_t k_sb, int64_t k_sh, int64_t k_si, const void* v, int64_t v_sb,
                                        int64_t v_sh, int64_t v_si, const uint8_t* valid, int64_t valid_sb,
                                        int32_t B, int32_t heads, int32_t n, int32_t head_dim, float scale,
                                        const float* o, int64_t o_sb, int64_t o_sh, int64_t o_si, const float* lse,
                                        int64_t l_sb, int64_t l_sh, const float* dout, int64_t d_sb, int64_t d_sh,
                                        int64_t d_si, const float* dlse, float* delta, float* dq, float* dk,
                                        float* dv, int64_t g_sb, int64_t g_sh, int64_t g_si, void* stream) {
  using namespace hla;
  HfChunkParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.q_sb = q_sb, p.q_sh = q_sh, p.q_si = q_si, p.k_sb = k_sb, p.k_sh = k_sh, p.k_si = k_si;
  p.v_sb = v_sb, p.v_sh = v_sh, p.v_si = v_si;
  p.valid = valid;
  p.valid_sb = valid_sb;
  p.n = n;
  p.scale = scale;
  p.scale_log2 = scale * kLog2e;
  p.o = const_cast<float*>(o), p.o_sb = o_sb, p.o_sh = o_sh, p.o_si = o_si;
  p.lse = const_cast<float*>(lse), p.l_sb = l_sb, p.l_sh = l_sh;
  p.dout = dout, p.d_sb = d_sb, p.d_sh = d_sh, p.d_si = d_si;
  p.dlse = dlse;
  p.delta = delta;
  p.dq = dq, p.dk = dk, p.dv = dv, p.g_sb = g_sb, p.g_sh = g_sh, p.g_si = g_si;
  if (B == 0 || n == 0) return HLA_S6_OK;
  int rc = check_operands(p, B, heads, head_dim, "hf_chunk_backward");
  if (rc != HLA_S6_OK) return rc;
  HLA_REQUIRE(dout && delta && dq && dk && dv, HLA_S6_EINVAL, "hf_chunk_backward: null pointer argument");
  HLA_REQUIRE(aligned16(dout) && d_sb % 4 == 0 && d_sh % 4 == 0 && d_si % 4 == 0 && aligned16(dq) && aligned16(dk) &&
                  aligned16(dv) && g_sb % 4 == 0 && g_sh % 4 == 0 && g_si % 4 == 0,
              HLA_S6_EINVAL, "hf_chunk_backward: dout / gradient rows must be 16-byte aligned");
  const dim3 grid((unsigned)((n + 15) / 16), kHF, (unsigned)B);
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(chunk_dq, grid, dim3(64), 0, st, p);  // also writes delta for chunk_dkdv
  rc = check_launch("hf_chunk_backward (dq)");
  if (rc != HLA_S6_OK) return rc;
  hipLaunchKernelGGL(chunk_dkdv, grid, dim3(64), 0, st, p);
  return check_launch("hf_chunk_backward (dk, dv)");
}
