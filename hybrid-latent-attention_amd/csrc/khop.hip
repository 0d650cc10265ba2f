// Multi-query latent history attention on contiguous rows with an arbitrary visibility mask, forward and backward
// (the K-hop replay / training form: hla/latent/history_gemm.py:159-220, hla/latent/fused_history.py:126-153).
//
//   q [B, Lq, 16, R], k/v [B, N, R] (rows shared by the 16 heads), mask [B, Lq, N] (nonzero = visible)
//   z[b,i,h] = softmax_j(scale q.k_j | visible) . v,  lse[b,h,i] (natural log; -inf and z = 0 with no visible key)
//   backward (P = exp(s - lse), delta = dz.z):  dv = P^T dz,  dS = P (dz.v - delta + dlse) scale,
//                                               dq = dS k,    dk = dS^T q
//
// Every kernel works on steps of 32 query rows (2 tokens x 16 heads) x 32 keys with 8 waves. The operand tiles sit
// in LDS (row-major, rows padded by 16 elements): score blocks S = Q K^T and dP = dZ V^T are 16 x 16 blocks on
// v_mfma_f32_16x16x32_bf16 with both operands read as 16-byte rows (k = latent column); the products over keys or
// rows (P V, dS K, P^T dZ, dS^T Q) take their k-contiguous operand from a small bf16 LDS block and the other one
// transposed by ds_read_b64_tr_b16, and split the R output columns over the 8 waves. P and dS enter the second
// products rounded to bf16 (bf16 operands, fp32 accumulation, as the reference's bf16 mode).
//
// Each token's key bound (1 + its last visible key, from the mask) limits the key range, so a causal mask costs
// half the work without a causality promise.
#include "common.h"

namespace hla {
namespace {


constexpr int kKhRows = 32;   // query rows per step (2 tokens x 16 heads)
constexpr int kKhKeys = 32;   // keys per step
constexpr int kKhThreads = 512;
constexpr int kKhPS = kKhKeys + 8;  // LDS row stride of the bf16 P / dS blocks

struct KhopParams {
  const uint16_t* q;
  int64_t q_sb, q_si, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sb, k_sn, v_sb, v_sn;
  const uint8_t* mask;  // may be null (then every key below the bound is visible)
  int64_t m_sb, m_si;
  const int32_t* bound;  // [B * Lq] keys below this are candidates
  int B, Lq, N;
  float scale, scale_log2;
  // forward outputs / backward inputs
  uint16_t* z;
  int64_t z_sb, z_si, z_sh;
  float* lse;  // [B, 16, Lq]
  const uint16_t* dz;
  int64_t dz_sb, dz_si, dz_sh;
  const float* dlse;   // [B, 16, Lq] or null
  const float* delta;  // [B, 16, Lq]
  // backward outputs (fp32)
  float* dq;
  int64_t dq_sb, dq_si, dq_sh;
  float* dk;
  float* dv;
  int64_t dk_sb, dk_sn, dv_sb, dv_sn;
  int key_splits;  // dkdv: row ranges per key tile (partials of split s go to dk + s * dk_ss)
  int64_t dk_ss, dv_ss;
  int64_t dq_ss;   // dq4 with key ranges (gridDim.z > 1): the partial of range z goes to dq + z * dq_ss
  bool dq_bf16, kv_bf16;  // the kernel writes dq (dk, dv) as bf16 (strides in bf16 elements) instead of fp32
};

// Gradient stores: fp32, or bf16 rounded to nearest even (the rounding of a torch cast) into a bf16 array whose
// element offset is i.
__device__ __forceinline__ void kh_store1(float* p, int64_t i, float v, bool bf) {
  if (bf) reinterpret_cast<uint16_t*>(p)[i] = f2bf(v);
  else p[i] = v;
}
__device__ __forceinline__ void kh_store4(float* p, int64_t i, floatx4 v, bool bf) {
  if (bf) *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p) + i) = uint2{pack2(v[0], v[1]), pack2(v[2], v[3])};
  else *reinterpret_cast<floatx4*>(p + i) = v;
}

template <int R>
struct KhGeo {
  static constexpr int RS = R + 16;           // LDS row stride of the operand tiles (bf16): rows 8 banks apart, so
                                              // 16-byte row reads and the transposing reads are conflict-free
  static constexpr int CPR = R / 8;           // 16-byte pieces per row
  static constexpr int TL = 32 * CPR / kKhThreads;  // pieces per thread per 32-row tile
  static constexpr int QW = R / 8;            // output columns per wave
  static constexpr int CB = QW / 16;          // 16-column blocks per wave
  static_assert(TL >= 1 && QW >= 16, "R must be at least 128");
};

// Load 32 rows x R of a row-major bf16 matrix into registers (coalesced: piece c = it * 512 + tid is row c / CPR,
// 16-byte piece c % CPR); rows are addressed by `rowp(r)` (a clamped, in-bounds row pointer).
template <int R, class RowP>
__device__ __forceinline__ void kh_load(u32x4 (&reg)[KhGeo<R>::TL], RowP rowp) {
  using G = KhGeo<R>;
#pragma unroll
  for (int it = 0; it < G::TL; ++it) {
    const int c = it * kKhThreads + threadIdx.x;
    reg[it] = ld16(rowp(c / G::CPR) + (c % G::CPR) * 8);
  }
}

template <int R>
__device__ __forceinline__ void kh_store(uint16_t* tile, const u32x4 (&reg)[KhGeo<R>::TL]) {
  using G = KhGeo<R>;
#pragma unroll
  for (int it = 0; it < G::TL; ++it) {
    const int c = it * kKhThreads + threadIdx.x;
    st16(tile + (c / G::CPR) * G::RS + (c % G::CPR) * 8, reg[it]);
  }
}

// 16 x 16 block D[m][n] = sum_c A[16 mb + m][c] * Bt[16 nb + n][c] over c in [c0, c1) of two row-major LDS tiles.
// Lane l holds D[4 (l / 16) + r][l % 16], r < 4.
template <int R>
__device__ __forceinline__ floatx4 kh_block(const uint16_t* A, int mb, const uint16_t* Bt, int nb, int c0, int c1) {
  using G = KhGeo<R>;
  const int lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
  const uint16_t* ap = A + (16 * mb + l16) * G::RS + 8 * g;
  const uint16_t* bp = Bt + (16 * nb + l16) * G::RS + 8 * g;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int c = c0; c < c1; c += 32)
    acc = mfma16x16x32(*reinterpret_cast<const u32x4*>(ap + c), *reinterpret_cast<const u32x4*>(bp + c), acc);
  return acc;
}

// Transposed B operand of a 16x16x32 product over 32 rows of a row-major LDS tile: lane (g, i) gets
// tile[8g + e][c0 + i] for e < 8 (two ds_read_b64_tr_b16, each moving 4 rows of one column per lane).
template <int R>
__device__ __forceinline__ u32x4 kh_tr(const uint16_t* tile, int c0) {
  using G = KhGeo<R>;
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const uint16_t* p = tile + (8 * g + (j >> 2)) * G::RS + c0 + 4 * (j & 3);
  const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)p);
  const short4v hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)(p + 4 * G::RS));
  return join_tr(lo, hi);
}

// out[16 mb .. +16][wave columns] += Pb[16 mb + m][k < 32] * T[k][col] (T a row-major LDS tile over 32 rows).
template <int R>
__device__ __forceinline__ void kh_accumulate(floatx4 (&acc)[2][KhGeo<R>::CB], const uint16_t* Pb,
                                              const uint16_t* T) {
  using G = KhGeo<R>;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  u32x4 pa[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) pa[mb] = *reinterpret_cast<const u32x4*>(Pb + (16 * mb + l16) * kKhPS + 8 * g);
#pragma unroll
  for (int cb = 0; cb < G::CB; ++cb) {
    const u32x4 tb = kh_tr<R>(T, wave * G::QW + 16 * cb);
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) acc[mb][cb] = mfma16x16x32(pa[mb], tb, acc[mb][cb]);
  }
}

// ---- row data loaded one step ahead ---------------------------------------------------------------------------
// What the P / dS role of thread (row sr, keys 2 kp, 2 kp + 1) needs from memory for one step: the row's lse,
// delta, dlse and key bound, and the mask bytes of its two keys. Loaded one step ahead (plain register loads, used
// after the next barrier), so their latency is not on the step's critical path.
struct KhRow {
  float lse, delta, dlse;
  int bound;
  uint8_t m[2];
};

__device__ __forceinline__ KhRow kh_row_load(const KhopParams& a, int b, int i, int h, int key0, int kp) {
  KhRow r;
  const int64_t idx = ((int64_t)b * 16 + h) * a.Lq + i, t = (int64_t)b * a.Lq + i;
  r.lse = a.lse[idx];
  r.delta = a.delta[idx];
  r.dlse = a.dlse ? a.dlse[idx] : 0.f;
  r.bound = a.bound[t];
  r.m[0] = r.m[1] = 1;
  if (a.mask) {
    const uint8_t* mr = a.mask + (int64_t)b * a.m_sb + (int64_t)i * a.m_si;
    r.m[0] = mr[min(key0 + 2 * kp, a.N - 1)];
    r.m[1] = mr[min(key0 + 2 * kp + 1, a.N - 1)];
  }
  return r;
}

// Mask bytes only (the dq kernel keeps its rows for the whole pass).
__device__ __forceinline__ void kh_mask_load(const KhopParams& a, int b, int i, int key0, int kp, uint8_t (&m)[2]) {
  m[0] = m[1] = 1;
  if (a.mask) {
    const uint8_t* mr = a.mask + (int64_t)b * a.m_sb + (int64_t)i * a.m_si;
    m[0] = mr[min(key0 + 2 * kp, a.N - 1)];
    m[1] = mr[min(key0 + 2 * kp + 1, a.N - 1)];
  }
}

// ---- forward -------------------------------------------------------------------------------------------------
// One workgroup per 2 consecutive tokens of a batch row: Q resident in LDS, K/V tiles of 32 keys streamed through
// LDS (the next tile's loads in flight in registers), online softmax per query row (16 lanes per row).
template <int R>
__global__ __launch_bounds__(kKhThreads) void khop_fwd(KhopParams a) {
  using G = KhGeo<R>;
  __shared__ __attribute__((aligned(16))) uint16_t qs[kKhRows * G::RS];
  __shared__ __attribute__((aligned(16))) uint16_t ks[kKhKeys * G::RS];
  __shared__ __attribute__((aligned(16))) uint16_t vs[kKhKeys * G::RS];
  __shared__ __attribute__((aligned(16))) floatx4 sx[8][64];
  __shared__ __attribute__((aligned(16))) uint16_t ps[kKhRows * kKhPS];
  __shared__ float alpha_s[kKhRows], l_s[kKhRows], m_s[kKhRows];
  __shared__ int bound_s[2];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int b = blockIdx.y, i0 = blockIdx.x * 2;
  const int64_t t0 = (int64_t)b * a.Lq + i0;
  const int ntok = min(2, a.Lq - i0);
  if (tid < 2) bound_s[tid] = tid < ntok ? min(a.bound[t0 + tid], a.N) : 0;
  {
    u32x4 qr[G::TL];
    kh_load<R>(qr, [&](int r) {
      const int tok = min(r >> 4, ntok - 1);
      return a.q + (int64_t)b * a.q_sb + (int64_t)(i0 + tok) * a.q_si + (int64_t)(r & 15) * a.q_sh;
    });
    kh_store<R>(qs, qr);
  }
  __syncthreads();
  const int nkeys = max(bound_s[0], bound_s[1]);
  // softmax role: row sr (token sr / 16, head sr % 16), keys 2 kp, 2 kp + 1
  const int sr = tid >> 4, kp = tid & 15;
  const int row_i = i0 + min(sr >> 4, ntok - 1);
  const int row_bound = a.bound[t0 + min(sr >> 4, ntok - 1)];
  uint8_t m_cur[2], m_next[2] = {1, 1};
  float m_run = -INFINITY, l_run = 0.f;
  floatx4 acc[2][G::CB];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int cb = 0; cb < G::CB; ++cb) acc[mb][cb] = floatx4{0.f, 0.f, 0.f, 0.f};

  u32x4 kr[G::TL], vr[G::TL];
  auto load_kv = [&](int kt) {
    kh_load<R>(kr, [&](int r) { return a.k + (int64_t)b * a.k_sb + (int64_t)min(kt + r, a.N - 1) * a.k_sn; });
    kh_load<R>(vr, [&](int r) { return a.v + (int64_t)b * a.v_sb + (int64_t)min(kt + r, a.N - 1) * a.v_sn; });
  };
  if (nkeys > 0) {
    load_kv(0);
    kh_mask_load(a, b, row_i, 0, kp, m_next);
  }
  for (int kt = 0; kt < nkeys; kt += kKhKeys) {
    __syncthreads();  // the previous step's readers of ks / vs / ps are done
    kh_store<R>(ks, kr);
    kh_store<R>(vs, vr);
    m_cur[0] = m_next[0];
    m_cur[1] = m_next[1];
    __syncthreads();
    if (kt + kKhKeys < nkeys) {
      load_kv(kt + kKhKeys);
      kh_mask_load(a, b, row_i, kt + kKhKeys, kp, m_next);
    }
    {  // S partials: wave w -> block w % 4 (rows 16 (w/2 % 2).., keys 16 (w % 2)..), column half w / 4
      const int blk = wave & 3, half = wave >> 2;
      sx[wave][lane] = kh_block<R>(qs, blk >> 1, ks, blk & 1, half * (R / 2), (half + 1) * (R / 2));
    }
    __syncthreads();
    {  // online softmax of row sr over keys kt + 2 kp, + 1
      const int rb = sr >> 4, r4 = sr & 15;
      float s2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int key = 2 * kp + e, blk = 2 * rb + (key >> 4);
        const int li = 16 * (r4 >> 2) + (key & 15);
        const float s = sx[blk][li][r4 & 3] + sx[blk + 4][li][r4 & 3];
        s2[e] = kt + key < row_bound && m_cur[e] && (sr >> 4) < ntok ? s * a.scale_log2 : -INFINITY;
      }
      float mx = fmaxf(s2[0], s2[1]);
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);  // m_run = -inf: alpha = 0
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float p0 = fast_exp2(s2[0] - m_use), p1 = fast_exp2(s2[1] - m_use);
      float ps_sum = p0 + p1;
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) ps_sum += __shfl_xor(ps_sum, off);
      l_run = l_run * alpha + ps_sum;
      m_run = m_new;
      *reinterpret_cast<uint32_t*>(ps + sr * kKhPS + 2 * kp) = pack2(p0, p1);
      if (kp == 0) alpha_s[sr] = alpha;
    }
    __syncthreads();
    {  // O = alpha O + P V over this wave's columns
      const int g = lane >> 4;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const floatx4 al = {alpha_s[16 * mb + 4 * g], alpha_s[16 * mb + 4 * g + 1], alpha_s[16 * mb + 4 * g + 2],
                            alpha_s[16 * mb + 4 * g + 3]};
#pragma unroll
        for (int cb = 0; cb < G::CB; ++cb) acc[mb][cb] *= al;
      }
      kh_accumulate<R>(acc, ps, vs);
    }
  }
  if (kp == 0) {
    l_s[sr] = l_run;
    m_s[sr] = m_run;
  }
  __syncthreads();
  {
    const int l16 = lane & 15, g = lane >> 4;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mb + 4 * g + r, tok = row >> 4, h = row & 15;
        if (tok >= ntok) continue;
        const float l = l_s[row];
        const float inv = l > 0.f ? 1.f / l : 0.f;
        uint16_t* zp = a.z + (int64_t)b * a.z_sb + (int64_t)(i0 + tok) * a.z_si + (int64_t)h * a.z_sh;
#pragma unroll
        for (int cb = 0; cb < G::CB; ++cb) zp[wave * G::QW + 16 * cb + l16] = f2bf(acc[mb][cb][r] * inv);
      }
    }
    if (tid < kKhRows && (tid >> 4) < ntok) {
      const float l = l_s[tid];
      a.lse[((int64_t)b * 16 + (tid & 15)) * a.Lq + i0 + (tid >> 4)] =
          l > 0.f ? (m_s[tid] + log2f(l)) * kLn2 : -INFINITY;
    }
  }
}

// ---- backward helpers ----------------------------------------------------------------------------------------
// Row constants of a query row: lse in the log2 domain (0 for a row without history: all its P are 0 anyway) and
// delta - dlse.
__device__ __forceinline__ void kh_row_consts(const KhRow& r, float& lse2, float& dd) {
  const bool empty = !(r.lse > -INFINITY);
  lse2 = empty ? 0.f : r.lse * kLog2e;
  dd = r.delta - (empty ? 0.f : r.dlse);
}

// bf16 of one finite fp32 value by the hardware conversion (round to nearest even)
__device__ __forceinline__ uint16_t f2bf_hw(float x) { return (uint16_t)pack2_hw(x, 0.f); }

// P and dS of a 32-row x 32-key step from the S blocks (waves 0-3) and dP blocks (waves 4-7) in sx, written as
// bf16 to pb / dsb in [row][key] order (kTransposed: [key][row]). Row constants of row sr: lse2 (log2 domain),
// delta - dlse in dd; key key0 + 2 kp + e is visible when row_ok, below the row's bound and its mask byte is set.
template <bool kTransposed>
__device__ __forceinline__ void kh_pds(const KhopParams& a, const floatx4 (*sx)[64], uint16_t* pb, uint16_t* dsb,
                                       int bound, const uint8_t (&m)[2], bool row_ok, int key0, float lse2,
                                       float dd) {
  const int tid = threadIdx.x, sr = tid >> 4, kp = tid & 15;
  const int rb = sr >> 4, r4 = sr & 15;
  float p[2], ds[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int key = 2 * kp + e, blk = 2 * rb + (key >> 4);
    const int li = 16 * (r4 >> 2) + (key & 15);
    const float s = sx[blk][li][r4 & 3], dp = sx[blk + 4][li][r4 & 3];
    const bool vis = row_ok && key0 + key < bound && m[e] != 0;
    p[e] = vis ? fast_exp2(s * a.scale_log2 - lse2) : 0.f;
    ds[e] = p[e] * (dp - dd) * a.scale;
  }
  if (kTransposed) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      pb[(2 * kp + e) * kKhPS + sr] = f2bf_hw(p[e]);
      dsb[(2 * kp + e) * kKhPS + sr] = f2bf_hw(ds[e]);
    }
  } else {
    *reinterpret_cast<uint32_t*>(pb + sr * kKhPS + 2 * kp) = pack2_hw(p[0], p[1]);
    *reinterpret_cast<uint32_t*>(dsb + sr * kKhPS + 2 * kp) = pack2_hw(ds[0], ds[1]);
  }
}

// ---- backward: dq ----------------------------------------------------------------------------------------------
template <int R>
__global__ __launch_bounds__(kKhThreads) void khop_dq(KhopParams a) {
  using G = KhGeo<R>;
  __shared__ __attribute__((aligned(16))) uint16_t qs[kKhRows * G::RS];
  __shared__ __attribute__((aligned(16))) uint16_t dzs[kKhRows * G::RS];
  __shared__ __attribute__((aligned(16))) uint16_t ks[kKhKeys * G::RS];
  __shared__ __attribute__((aligned(16))) uint16_t vs[kKhKeys * G::RS];
  __shared__ __attribute__((aligned(16))) floatx4 sx[8][64];
  __shared__ __attribute__((aligned(16))) uint16_t pb[kKhRows * kKhPS];
  __shared__ __attribute__((aligned(16))) uint16_t dsb[kKhRows * kKhPS];
  __shared__ int bound_s[2];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int b = blockIdx.y, i0 = blockIdx.x * 2;
  const int64_t t0 = (int64_t)b * a.Lq + i0;
  const int ntok = min(2, a.Lq - i0);
  if (tid < 2) bound_s[tid] = tid < ntok ? min(a.bound[t0 + tid], a.N) : 0;
  {
    u32x4 r0[G::TL];
    kh_load<R>(r0, [&](int r) {
      const int tok = min(r >> 4, ntok - 1);
      return a.q + (int64_t)b * a.q_sb + (int64_t)(i0 + tok) * a.q_si + (int64_t)(r & 15) * a.q_sh;
    });
    kh_store<R>(qs, r0);
    kh_load<R>(r0, [&](int r) {
      const int tok = min(r >> 4, ntok - 1);
      return a.dz + (int64_t)b * a.dz_sb + (int64_t)(i0 + tok) * a.dz_si + (int64_t)(r & 15) * a.dz_sh;
    });
    kh_store<R>(dzs, r0);
  }
  __syncthreads();
  const int nkeys = max(bound_s[0], bound_s[1]);
  const int sr = tid >> 4, kp = tid & 15;
  const bool row_ok = (sr >> 4) < ntok;
  const int row_i = i0 + min(sr >> 4, ntok - 1);
  const KhRow row = kh_row_load(a, b, row_i, sr & 15, 0, kp);
  float lse2, dd;
  kh_row_consts(row, lse2, dd);
  uint8_t m_cur[2] = {row.m[0], row.m[1]}, m_next[2] = {1, 1};
  floatx4 acc[2][G::CB];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int cb = 0; cb < G::CB; ++cb) acc[mb][cb] = floatx4{0.f, 0.f, 0.f, 0.f};
  u32x4 kr[G::TL], vr[G::TL];
  auto load_kv = [&](int kt) {
    kh_load<R>(kr, [&](int r) { return a.k + (int64_t)b * a.k_sb + (int64_t)min(kt + r, a.N - 1) * a.k_sn; });
    kh_load<R>(vr, [&](int r) { return a.v + (int64_t)b * a.v_sb + (int64_t)min(kt + r, a.N - 1) * a.v_sn; });
  };
  if (nkeys > 0) load_kv(0);
  for (int kt = 0; kt < nkeys; kt += kKhKeys) {
    __syncthreads();
    kh_store<R>(ks, kr);
    kh_store<R>(vs, vr);
    __syncthreads();
    if (kt + kKhKeys < nkeys) {
      load_kv(kt + kKhKeys);
      kh_mask_load(a, b, row_i, kt + kKhKeys, kp, m_next);
    }
    {  // waves 0-3: S block w; waves 4-7: dP block w - 4 (full R)
      const int blk = wave & 3;
      sx[wave][lane] = wave < 4 ? kh_block<R>(qs, blk >> 1, ks, blk & 1, 0, R)
                                : kh_block<R>(dzs, blk >> 1, vs, blk & 1, 0, R);
    }
    __syncthreads();
    kh_pds<false>(a, sx, pb, dsb, row.bound, m_cur, row_ok, kt, lse2, dd);
    m_cur[0] = m_next[0];
    m_cur[1] = m_next[1];
    __syncthreads();
    kh_accumulate<R>(acc, dsb, ks);  // dQ += dS K
  }
  {
    const int l16 = lane & 15, g = lane >> 4;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mb + 4 * g + r, tok = row >> 4, h = row & 15;
        if (tok >= ntok) continue;
        const int64_t o = (int64_t)b * a.dq_sb + (int64_t)(i0 + tok) * a.dq_si + (int64_t)h * a.dq_sh;
#pragma unroll
        for (int cb = 0; cb < G::CB; ++cb)
          kh_store1(a.dq, o + wave * G::QW + 16 * cb + l16, acc[mb][cb][r], a.dq_bf16);
      }
  }
}

// ---- backward: dq on the multi-query layout ---------------------------------------------------------------
// khop_dq4: one workgroup per 4 consecutive tokens of a batch row, 8 waves; wave w serves token w / 2 and, for the
// score blocks, role w % 2: role 0 computes S^T = K Q^T and role 1 dP^T = V dZ^T over all R columns (the token's
// Q^T or dZ^T in registers as the MFMA B operand, the 16-byte K or V rows of the tile as the A operand). The pair
// swaps the two 32-key x 16-row blocks through LDS; both waves then form P = exp(S scale - lse) and
// dS = P (dP - delta + dlse) scale for the row of lane l % 16, keep dS^T in registers as the B operand (the score
// layout is that operand's layout under a fixed permutation of the 32 keys over the MFMA k index, which the two
// transposing reads of K^T follow) and accumulate dQ^T over their column half (R / 2) from K^T fragments.
// K and V tiles of 32 keys go global -> LDS by direct copies into four buffers (K and V of tiles i and i + 1):
// after the swap barrier V(i+2) replaces V(i), after the dQ barrier K(i+2) replaces K(i), so every copy has about
// a tile of time; the copies are waited for by explicit s_waitcnt behind plain barriers. With a mask the 32 bytes of
// the wave's token for the tile travel with the K copy.
template <int R, bool kMask>
__global__ __launch_bounds__(kKhThreads, 1) void khop_dq4(KhopParams a) {
  constexpr int C = R / 2, KF = R / 32, CB = C / 16, RS = R + 16;
  constexpr int KOPS = kMask ? 5 : 4;  // copy instructions per wave for a K tile (4 rows, and the mask bytes)
  __shared__ __attribute__((aligned(16))) uint16_t kt_lds[2][32 * RS];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[2][32 * RS];
  __shared__ __attribute__((aligned(16))) floatx4 xs[8][2][64];      // [wave][key block][lane]
  __shared__ __attribute__((aligned(16))) uint8_t mk_lds[2][8][32];  // [tile parity][wave][key]
  __shared__ int bound_s[4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int u = wave >> 1, role = wave & 1, col0 = role * C;
  // token groups dispatched last to first: under a causal mask the last tokens see the most keys, so the longest
  // workgroups start first and the tail of the launch is short
  const int b = blockIdx.y, i0 = (gridDim.x - 1 - blockIdx.x) * 4;
  const int ntok = min(4, a.Lq - i0);
  const int iu = i0 + min(u, ntok - 1);  // this wave's token (clamped: waves past the last token store nothing)
  if (tid < 4) bound_s[tid] = tid < ntok ? min(a.bound[(int64_t)b * a.Lq + i0 + tid], a.N) : 0;
  // row constants of row (token iu, head l16): lse in the log2 domain (0 without history) and delta - dlse
  const int64_t ridx = ((int64_t)b * 16 + l16) * a.Lq + iu;
  const float lse = a.lse[ridx];
  const bool empty = !(lse > -INFINITY);
  const float lse2 = empty ? 0.f : lse * kLog2e;
  const float dd = a.delta[ridx] - (a.dlse && !empty ? a.dlse[ridx] : 0.f);
  u32x4 rf[KF];  // Q^T (role 0) or dZ^T (role 1) of the token: B operand, 8 consecutive columns per lane and k-step
  {
    const uint16_t* rp = role == 0
                             ? a.q + (int64_t)b * a.q_sb + (int64_t)iu * a.q_si + (int64_t)l16 * a.q_sh + 8 * g
                             : a.dz + (int64_t)b * a.dz_sb + (int64_t)iu * a.dz_si + (int64_t)l16 * a.dz_sh + 8 * g;
#pragma unroll
    for (int k = 0; k < KF; ++k) rf[k] = ld16(rp + 32 * k);
  }
  __syncthreads();
  const int nkeys = max(max(bound_s[0], bound_s[1]), max(bound_s[2], bound_s[3]));
  const int own_bound = bound_s[min(u, ntok - 1)];
  // key range z of gridDim.z: tiles [tb, te) of the workgroup's 32-key tiles (dq is linear in the keys, so each
  // range writes a partial and the partials are summed afterwards)
  // (uniform, and kept in SGPRs: the copy instructions take the tile's row address and LDS buffer from them)
  const int tiles_all = (nkeys + 31) / 32;
  const int per = (tiles_all + (int)gridDim.z - 1) / (int)gridDim.z;
  const int tb = __builtin_amdgcn_readfirstlane(min(tiles_all, (int)blockIdx.z * per));
  const int te = __builtin_amdgcn_readfirstlane(min(tiles_all, tb + per));
  // every earlier load is complete before the first copy: the compiler does not see the copies, so no wait it
  // places for an earlier load may end up counting them
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
  floatx4 acc[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) acc[cb] = floatx4{0.f, 0.f, 0.f, 0.f};
  const uint32_t voff = 16u * lane;
  // rows 4 * wave .. + 3 of the tile at key kt (keys past N read row N - 1)
  auto copy_rows = [&](uint16_t* buf, const uint16_t* base, int64_t bst, int64_t rst, int kt) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int r = 4 * wave + r4;
      const uint16_t* row = base + (int64_t)b * bst + (int64_t)min(kt + r, a.N - 1) * rst;
      if (R == 512 || lane < 32) copy16_to_lds_rfl(row, voff, &buf[r * RS]);
    }
  };
  auto copy_k = [&](int j) {  // K tile j, and the mask bytes of this wave's token for it (lanes 0-1)
    const int kt = j * 32;
    if (kMask && lane < 2) {
      const int c0 = min(kt + 16 * lane, a.N - 16);  // N is a multiple of 16; keys past N are past every bound
      copy16_to_lds_v(a.mask + (int64_t)b * a.m_sb + (int64_t)iu * a.m_si + c0, &mk_lds[j & 1][wave][0]);
    }
    copy_rows(kt_lds[j & 1], a.k, a.k_sb, a.k_sn, kt);
  };
  auto copy_v = [&](int j) { copy_rows(vt_lds[j & 1], a.v, a.v_sb, a.v_sn, j * 32); };

  if (tb < te) {
    copy_k(tb);
    copy_v(tb);
    if (te - tb > 1) {
      copy_k(tb + 1);
      copy_v(tb + 1);
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(KOPS + 4, 15));  // tile tb landed; tile tb+1 may be in flight
    } else {
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
    }
    plain_barrier();
  }
  for (int i = tb; i < te; ++i) {
    const int kt = i * 32, par = i & 1;
    const bool more = i + 1 < te, more2 = i + 2 < te;
    floatx4 sb[2];  // this wave's block: S^T (role 0) or dP^T (role 1), keys kt + 16 kb + 4g + r, row l16
    {
      const uint16_t* ap = (role == 0 ? kt_lds[par] : vt_lds[par]) + l16 * RS + 8 * g;
      sb[0] = sb[1] = floatx4{0.f, 0.f, 0.f, 0.f};
      u32x4 fa = *reinterpret_cast<const u32x4*>(ap), fc = *reinterpret_cast<const u32x4*>(ap + 16 * RS);
#pragma unroll
      for (int k = 0; k < KF; ++k) {  // the next k-step's fragments are requested before this one's MFMAs
        const u32x4 ca = fa, cc = fc;
        if (k + 1 < KF) {
          fa = *reinterpret_cast<const u32x4*>(ap + 32 * (k + 1));
          fc = *reinterpret_cast<const u32x4*>(ap + 16 * RS + 32 * (k + 1));
        }
        sb[0] = mfma16x16x32(ca, rf[k], sb[0]);
        sb[1] = mfma16x16x32(cc, rf[k], sb[1]);
      }
    }
    xs[wave][0][lane] = sb[0];
    xs[wave][1][lane] = sb[1];
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));  // the block is in LDS
    plain_barrier();
    if (more2) copy_v(i + 2);  // V(i+2) into V(i)'s buffer: every wave is past its score block
    const floatx4 ob0 = xs[wave ^ 1][0][lane], ob1 = xs[wave ^ 1][1][lane];
    const floatx4 s0 = role == 0 ? sb[0] : ob0, s1 = role == 0 ? sb[1] : ob1;
    const floatx4 d0 = role == 0 ? ob0 : sb[0], d1 = role == 0 ? ob1 : sb[1];
    uint32_t m0 = ~0u, m1 = ~0u;
    if (kMask) {
      const uint8_t* mb = &mk_lds[par][wave][4 * g];
      m0 = *reinterpret_cast<const uint32_t*>(mb);
      m1 = *reinterpret_cast<const uint32_t*>(mb + 16);
    }
    float ds[2][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool v0 = kt + 4 * g + r < own_bound && ((m0 >> (8 * r)) & 255u) != 0;
      const bool v1 = kt + 16 + 4 * g + r < own_bound && ((m1 >> (8 * r)) & 255u) != 0;
      const float p0 = v0 ? fast_exp2(s0[r] * a.scale_log2 - lse2) : 0.f;
      const float p1 = v1 ? fast_exp2(s1[r] * a.scale_log2 - lse2) : 0.f;
      ds[0][r] = p0 * (d0[r] - dd) * a.scale;
      ds[1][r] = p1 * (d1[r] - dd) * a.scale;
    }
    const u32x4 dsb = {pack2_hw(ds[0][0], ds[0][1]), pack2_hw(ds[0][2], ds[0][3]), pack2_hw(ds[1][0], ds[1][1]),
                       pack2_hw(ds[1][2], ds[1][3])};
    {  // dQ^T += K^T dS^T over this wave's columns (k slot 8g + e <-> key 4g + e, e < 4; 16 + 4g + e - 4, e >= 4)
      const uint16_t* kp = &kt_lds[par][(4 * g + (l16 >> 2)) * RS + col0 + 4 * (l16 & 3)];
      auto kfrag = [&](int cb) {
        const short4v lo =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)(kp + 16 * cb));
        const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) short4v*)(kp + 16 * RS + 16 * cb));
        return join_tr(lo, hi);
      };
      u32x4 kf = kfrag(0);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const u32x4 cur = kf;
        if (cb + 1 < CB) kf = kfrag(cb + 1);
        acc[cb] = mfma16x16x32(cur, dsb, acc[cb]);
      }
    }
    if (more) {
      // tile i+1 landed (only V(i+2) may still be in flight); every wave is done with K(i) and the blocks
      if (more2) __builtin_amdgcn_s_waitcnt(waitcnt_imm(4, 0));
      else __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
      plain_barrier();
      if (more2) copy_k(i + 2);  // K(i+2) into K(i)'s buffer
    }
  }
  if (u < ntok) {  // lane holds dQ^T[col 16cb + 4g + r][head l16] of token i0 + u
    const int64_t o = blockIdx.z * a.dq_ss + (int64_t)b * a.dq_sb + (int64_t)(i0 + u) * a.dq_si +
                      (int64_t)l16 * a.dq_sh + col0 + 4 * g;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) kh_store4(a.dq, o + 16 * cb, acc[cb], a.dq_bf16);
  }
}

// ---- backward: dk, dv ----------------------------------------------------------------------------------------
// One workgroup per (32-key tile of a batch row, row split): K/V tile resident in LDS, the query rows of the split
// streamed in steps of 2 tokens (Q and dZ through LDS, the next step's loads in flight in registers); steps whose
// tokens cannot see the tile are skipped.
template <int R>
__global__ __launch_bounds__(kKhThreads) void khop_dkdv(KhopParams a) {
  using G = KhGeo<R>;
  __shared__ __attribute__((aligned(16))) uint16_t qs[kKhRows * G::RS];
  __shared__ __attribute__((aligned(16))) uint16_t dzs[kKhRows * G::RS];
  __shared__ __attribute__((aligned(16))) uint16_t ks[kKhKeys * G::RS];
  __shared__ __attribute__((aligned(16))) uint16_t vs[kKhKeys * G::RS];
  __shared__ __attribute__((aligned(16))) floatx4 sx[8][64];
  __shared__ __attribute__((aligned(16))) uint16_t pt[kKhKeys * kKhPS];
  __shared__ __attribute__((aligned(16))) uint16_t dst[kKhKeys * kKhPS];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int b = blockIdx.y, kt = blockIdx.x * kKhKeys, split = blockIdx.z;
  const int steps = (a.Lq + 1) / 2;
  const int per = (steps + a.key_splits - 1) / a.key_splits;
  const int s_begin = split * per, s_end = min(steps, s_begin + per);
  {
    u32x4 r0[G::TL];
    kh_load<R>(r0, [&](int r) { return a.k + (int64_t)b * a.k_sb + (int64_t)min(kt + r, a.N - 1) * a.k_sn; });
    kh_store<R>(ks, r0);
    kh_load<R>(r0, [&](int r) { return a.v + (int64_t)b * a.v_sb + (int64_t)min(kt + r, a.N - 1) * a.v_sn; });
    kh_store<R>(vs, r0);
  }
  floatx4 dk_acc[2][G::CB], dv_acc[2][G::CB];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int cb = 0; cb < G::CB; ++cb) dk_acc[mb][cb] = dv_acc[mb][cb] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int sr = tid >> 4, kp = tid & 15;
  u32x4 qr[G::TL], dzr[G::TL];
  KhRow row_next;
  auto load_rows = [&](int step) {
    const int i0 = 2 * step, ntok = min(2, a.Lq - i0);
    kh_load<R>(qr, [&](int r) {
      const int tok = min(r >> 4, ntok - 1);
      return a.q + (int64_t)b * a.q_sb + (int64_t)(i0 + tok) * a.q_si + (int64_t)(r & 15) * a.q_sh;
    });
    kh_load<R>(dzr, [&](int r) {
      const int tok = min(r >> 4, ntok - 1);
      return a.dz + (int64_t)b * a.dz_sb + (int64_t)(i0 + tok) * a.dz_si + (int64_t)(r & 15) * a.dz_sh;
    });
    row_next = kh_row_load(a, b, i0 + min(sr >> 4, ntok - 1), sr & 15, kt, kp);
  };
  auto sees_tile = [&](int step) {  // either token of the step has candidate keys in this tile
    const int i0 = 2 * step;
    const int64_t t = (int64_t)b * a.Lq + i0;
    return a.bound[t] > kt || (i0 + 1 < a.Lq && a.bound[t + 1] > kt);
  };
  int step = s_begin;
  while (step < s_end && !sees_tile(step)) ++step;
  if (step < s_end) load_rows(step);
  while (step < s_end) {
    const int i0 = 2 * step, ntok = min(2, a.Lq - i0);
    __syncthreads();  // previous step's readers of qs / dzs / pt / dst are done
    kh_store<R>(qs, qr);
    kh_store<R>(dzs, dzr);
    const KhRow row = row_next;
    __syncthreads();
    int next = step + 1;
    while (next < s_end && !sees_tile(next)) ++next;
    if (next < s_end) load_rows(next);
    {
      const int blk = wave & 3;
      sx[wave][lane] = wave < 4 ? kh_block<R>(qs, blk >> 1, ks, blk & 1, 0, R)
                                : kh_block<R>(dzs, blk >> 1, vs, blk & 1, 0, R);
    }
    __syncthreads();
    {
      float lse2, dd;
      kh_row_consts(row, lse2, dd);
      kh_pds<true>(a, sx, pt, dst, row.bound, row.m, (sr >> 4) < ntok, kt, lse2, dd);
    }
    __syncthreads();
    kh_accumulate<R>(dv_acc, pt, dzs);  // dV += P^T dZ
    kh_accumulate<R>(dk_acc, dst, qs);  // dK += dS^T Q
    step = next;
  }
  {
    const int l16 = lane & 15, g = lane >> 4;
    const int64_t ok = split * a.dk_ss + (int64_t)b * a.dk_sb, ov = split * a.dv_ss + (int64_t)b * a.dv_sb;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kt + 16 * mb + 4 * g + r;
        if (key >= a.N) continue;
#pragma unroll
        for (int cb = 0; cb < G::CB; ++cb) {
          const int col = wave * G::QW + 16 * cb + l16;
          kh_store1(a.dk, ok + (int64_t)key * a.dk_sn + col, dk_acc[mb][cb][r], a.kv_bf16);
          kh_store1(a.dv, ov + (int64_t)key * a.dv_sn + col, dv_acc[mb][cb][r], a.kv_bf16);
        }
      }
  }
}

// ---- backward: dk, dv on the multi-query layout ----------------------------------------------------------
// khop_dkdv4: one workgroup per (64-key tile of a batch row, row split), 8 waves; wave w serves the 16 keys
// 16 (w / 2) .. of the tile and role w % 2: role 0 computes the score blocks S = Q K^T and accumulates dK^T, role 1
// the blocks dP = dZ V^T and dV^T. The wave's K^T or V^T (all R columns) stays in registers as the MFMA B operand;
// the query tokens of the split stream through LDS two at a time (32 rows): per step the pair swaps its two
// 32-row x 16-key blocks through LDS, both waves form P = exp(S scale - lse) and dS = P (dP - delta + dlse) scale
// (lane l holds rows 4 (l / 16) .. + 3 of each token for key l % 16: the B-operand layout of a 16x16x32 MFMA over
// the 32 rows under a fixed permutation of k, which the two transposing reads of the A operand follow), and role 0
// adds Q^T dS, role 1 dZ^T P over all R columns. Every step's Q and dZ rows, its rows' lse / delta / dlse and the
// tokens' key bounds (gathers of words) and the wave's mask bytes go global -> LDS by direct copies into two
// buffers, requested one step ahead. Tokens of the split before the first one whose bound reaches the tile are
// skipped; later tokens that see no key of the tile add zeros.
template <int R, bool kMask>
__global__ __launch_bounds__(kKhThreads, 1) void khop_dkdv4(KhopParams a) {
  constexpr int KF = R / 32, CBO = R / 16, RS = R + 16;
  constexpr int OPS = kMask ? 11 : 10;  // copies per wave per step: 8 rows, 2 gathers, the mask bytes
  __shared__ __attribute__((aligned(16))) uint16_t rows_lds[2][2][32 * RS];  // [buffer][Q, dZ][token * 16 + head]
  __shared__ __attribute__((aligned(16))) floatx4 xs[8][2][64];             // score blocks [wave][token][lane]
  // [buffer][wave][lse t0 | lse t1 | delta t0 | delta t1 | dlse t0 | dlse t1 | bound t0, t1]
  __shared__ __attribute__((aligned(16))) float rc_lds[2][8][128];
  __shared__ __attribute__((aligned(16))) uint8_t mk_lds[2][8][32];  // [buffer][wave][token * 16 + key of block]
  __shared__ int first_s;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int kb = wave >> 1, role = wave & 1;
  const int b = blockIdx.y, kt0 = blockIdx.x * 64, split = blockIdx.z;
  const int key = kt0 + 16 * kb + l16;  // this lane's key (clamped below for reads)
  const int keyc = min(key, a.N - 1);
  const int per = (a.Lq + a.key_splits - 1) / a.key_splits;
  const int s_begin = split * per, s_end = min(a.Lq, s_begin + per);
  // first token of the split whose key bound reaches the tile (bounds are arbitrary: every thread scans a share)
  if (tid == 0) first_s = s_end;
  __syncthreads();
  for (int i = s_begin + tid; i < s_end; i += kKhThreads)
    if (a.bound[(int64_t)b * a.Lq + i] > kt0) {
      atomicMin(&first_s, i);
      break;
    }
  u32x4 rf[KF];  // K^T (role 0) or V^T (role 1) of the wave's 16 keys: B operand
  {
    const uint16_t* rp = role == 0 ? a.k + (int64_t)b * a.k_sb + (int64_t)keyc * a.k_sn + 8 * g
                                   : a.v + (int64_t)b * a.v_sb + (int64_t)keyc * a.v_sn + 8 * g;
#pragma unroll
    for (int k = 0; k < KF; ++k) rf[k] = ld16(rp + 32 * k);
  }
  __syncthreads();
  const int first = __builtin_amdgcn_readfirstlane(first_s);
  // every earlier load is complete before the first copy: the compiler does not see the copies, so no wait it
  // places for an earlier load may end up counting them
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
  floatx4 acc[CBO];
#pragma unroll
  for (int cb = 0; cb < CBO; ++cb) acc[cb] = floatx4{0.f, 0.f, 0.f, 0.f};
  const uint32_t voff = 16u * lane;
  auto copy_step = [&](int i, int c) {  // tokens i, i + 1 (clamped to the split) into buffer c
    {  // 8 rows: waves 0-3 Q rows 8 (w % 4) .. + 7 of the step, waves 4-7 the dZ rows
      const int half = wave >> 2;
#pragma unroll
      for (int r8 = 0; r8 < 8; ++r8) {
        const int r = 8 * (wave & 3) + r8, tok = min(i + (r >> 4), s_end - 1), h = r & 15;
        const uint16_t* row = reinterpret_cast<const uint16_t*>(uniform64(
            half == 0 ? (int64_t)(a.q + (int64_t)b * a.q_sb + (int64_t)tok * a.q_si + (int64_t)h * a.q_sh)
                      : (int64_t)(a.dz + (int64_t)b * a.dz_sb + (int64_t)tok * a.dz_si + (int64_t)h * a.dz_sh)));
        if (R == 512 || lane < 32) copy16_to_lds(row, voff, &rows_lds[c][half][r * RS]);
      }
    }
    const int t1 = min(i + 1, s_end - 1);
    {  // lanes 0-15 / 16-31: lse of the two tokens, 32-47 / 48-63: their delta
      const int tok = (lane & 16) ? t1 : i, h = l16;
      const int64_t ridx = ((int64_t)b * 16 + h) * a.Lq + tok;
      copy4_to_lds_v(lane < 32 ? (const void*)(a.lse + ridx) : (const void*)(a.delta + ridx), &rc_lds[c][wave][0]);
    }
    if (lane < 34) {  // lanes 0-31: dlse of the two tokens (lse again without one), 32-33: their key bounds
      const int tok = (lane < 32 ? (lane & 16) : (lane & 1)) ? t1 : i, h = l16;
      const int64_t ridx = ((int64_t)b * 16 + h) * a.Lq + tok;
      copy4_to_lds_v(lane < 32 ? (const void*)(a.dlse ? a.dlse + ridx : a.lse + ridx)
                               : (const void*)(a.bound + (int64_t)b * a.Lq + tok),
                     &rc_lds[c][wave][64]);
    }
    if (kMask && lane < 2)
      copy16_to_lds_v(a.mask + (int64_t)b * a.m_sb + (int64_t)(lane ? t1 : i) * a.m_si +
                          min(kt0 + 16 * kb, a.N - 16),
                      &mk_lds[c][wave][0]);
  };
  const int nsteps = s_end > first ? (s_end - first + 1) / 2 : 0;
  if (nsteps > 0) {
    copy_step(first, 0);
    if (nsteps > 1) {
      copy_step(first + 2, 1);
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(OPS, 15));  // step 0 landed; step 1 may be in flight
    } else {
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
    }
    plain_barrier();
  }
  for (int j = 0; j < nsteps; ++j) {
    const int i = first + 2 * j, c = j & 1;
    const bool tok1 = i + 1 < s_end;  // the step's second token exists
    floatx4 sblk[2];  // S (role 0) or dP (role 1) of token x: rows 4g + r of key l16
    {
      const uint16_t* ap = &rows_lds[c][role][l16 * RS + 8 * g];  // A operand: Q or dZ rows l16, 16 + l16
      sblk[0] = sblk[1] = floatx4{0.f, 0.f, 0.f, 0.f};
      u32x4 fa = *reinterpret_cast<const u32x4*>(ap), fc = *reinterpret_cast<const u32x4*>(ap + 16 * RS);
#pragma unroll
      for (int k = 0; k < KF; ++k) {  // the next fragments are requested before this k-step's MFMAs
        const u32x4 ca = fa, cc = fc;
        if (k + 1 < KF) {
          fa = *reinterpret_cast<const u32x4*>(ap + 32 * (k + 1));
          fc = *reinterpret_cast<const u32x4*>(ap + 16 * RS + 32 * (k + 1));
        }
        sblk[0] = mfma16x16x32(ca, rf[k], sblk[0]);
        sblk[1] = mfma16x16x32(cc, rf[k], sblk[1]);
      }
    }
    xs[wave][0][lane] = sblk[0];
    xs[wave][1][lane] = sblk[1];
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));  // the blocks are in LDS
    plain_barrier();
    const float* rc = rc_lds[c][wave];
    float pq[2][4];  // P (role 1) or dS (role 0) of rows 4g + r of token x
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const floatx4 ob = xs[wave ^ 1][x][lane];
      const floatx4 sv = role == 0 ? sblk[x] : ob, dpv = role == 0 ? ob : sblk[x];
      const floatx4 lse4 = *reinterpret_cast<const floatx4*>(rc + 16 * x + 4 * g);
      const floatx4 del4 = *reinterpret_cast<const floatx4*>(rc + 32 + 16 * x + 4 * g);
      const floatx4 dl4 = *reinterpret_cast<const floatx4*>(rc + 64 + 16 * x + 4 * g);
      const int bnd = __float_as_int(rc[96 + x]);
      const bool vis = (x == 0 || tok1) && key < bnd && (!kMask || mk_lds[c][wave][16 * x + l16] != 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool emp = !(lse4[r] > -INFINITY);
        const float p = vis && !emp ? fast_exp2(sv[r] * a.scale_log2 - lse4[r] * kLog2e) : 0.f;
        const float dd = del4[r] - (a.dlse && !emp ? dl4[r] : 0.f);
        pq[x][r] = role == 0 ? p * (dpv[r] - dd) * a.scale : p;
      }
    }
    const u32x4 bq = {pack2_hw(pq[0][0], pq[0][1]), pack2_hw(pq[0][2], pq[0][3]), pack2_hw(pq[1][0], pq[1][1]),
                      pack2_hw(pq[1][2], pq[1][3])};
    {  // role 0: dK^T += Q^T dS; role 1: dV^T += dZ^T P (k slot 8g + e <-> row 4g + e of token 0, e < 4; of
       // token 1, e >= 4)
      const uint16_t* tp = &rows_lds[c][role][(4 * g + (l16 >> 2)) * RS + 4 * (l16 & 3)];
      auto afrag = [&](int cb) {
        const short4v lo =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)(tp + 16 * cb));
        const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) short4v*)(tp + 16 * RS + 16 * cb));
        return join_tr(lo, hi);
      };
      u32x4 af = afrag(0);
#pragma unroll
      for (int cb = 0; cb < CBO; ++cb) {
        const u32x4 cur = af;
        if (cb + 1 < CBO) af = afrag(cb + 1);
        acc[cb] = mfma16x16x32(cur, bq, acc[cb]);
      }
    }
    if (j + 1 < nsteps) {
      // step j+1 landed (nothing newer is in flight); every wave is done with buffer c
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
      plain_barrier();
      if (j + 2 < nsteps) copy_step(i + 4, c);  // step j+2 into step j's buffer
    }
  }
  if (key < a.N) {  // lane holds dK^T (role 0) or dV^T (role 1) [col 16 cb + 4g + r][key]
    float* out = role == 0 ? a.dk : a.dv;
    const int64_t o = role == 0 ? split * a.dk_ss + (int64_t)b * a.dk_sb + (int64_t)key * a.dk_sn
                                : split * a.dv_ss + (int64_t)b * a.dv_sb + (int64_t)key * a.dv_sn;
#pragma unroll
    for (int cb = 0; cb < CBO; ++cb) kh_store4(out, o + 16 * cb + 4 * g, acc[cb], a.kv_bf16);
  }
}

// ---- small kernels -------------------------------------------------------------------------------------------
// bound[t] = 1 + the last key mask row t shows (0 when none; N without a mask). One wave per row.
__global__ __launch_bounds__(256) void khop_bound_kernel(const uint8_t* mask, int64_t m_sb, int64_t m_si, int B,
                                                          int Lq, int N, int32_t* bound) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= (int64_t)B * Lq) return;
  if (!mask) {
    if (lane == 0) bound[t] = N;
    return;
  }
  const uint8_t* row = mask + (t / Lq) * m_sb + (t % Lq) * m_si;
  // the bytes before the row's first 16-byte boundary, then whole 16-byte words (all in flight at once), then the
  // tail; the highest nonzero byte of a little-endian word w is byte (31 - clz(w)) / 8
  const int head = min(N, (int)((16u - (reinterpret_cast<uintptr_t>(row) & 15u)) & 15u));
  const int nch = (N - head) >> 4, tail0 = head + 16 * nch;
  int last = -1;
  if (lane < head && row[lane]) last = lane;
  const u32x4* body = reinterpret_cast<const u32x4*>(row + head);
#pragma unroll 4
  for (int c = lane; c < nch; c += 64) {
    const u32x4 w = __builtin_nontemporal_load(body + c);
    const int base = head + 16 * c;
    if (w[3]) last = base + 12 + (31 - __clz(w[3])) / 8;
    else if (w[2]) last = base + 8 + (31 - __clz(w[2])) / 8;
    else if (w[1]) last = base + 4 + (31 - __clz(w[1])) / 8;
    else if (w[0]) last = base + (31 - __clz(w[0])) / 8;
  }
  if (tail0 + lane < N && row[tail0 + lane]) last = tail0 + lane;  // the tail is shorter than 16 bytes
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) last = max(last, __shfl_xor(last, off));
  if (lane == 0) bound[t] = last + 1;
}

// delta[b, h, i] = sum_c dz[b, i, h, c] * z[b, i, h, c] (fp32 products of the bf16 values). One wave per row.
__global__ __launch_bounds__(256) void khop_delta_kernel(const uint16_t* dz, int64_t dz_sb, int64_t dz_si,
                                                          int64_t dz_sh, const uint16_t* z, int64_t z_sb, int64_t z_si,
                                                          int64_t z_sh, int B, int Lq, int R, float* delta) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= (int64_t)B * Lq * 16) return;
  const int h = (int)(row % 16);
  const int64_t t = row / 16;
  const int b = (int)(t / Lq), i = (int)(t % Lq);
  const uint16_t* dzp = dz + b * dz_sb + i * dz_si + h * dz_sh;
  const uint16_t* zp = z + b * z_sb + i * z_si + h * z_sh;
  float s = 0.f;
  if ((((uintptr_t)dzp | (uintptr_t)zp) & 15u) == 0 && R % 8 == 0) {  // 8 columns per lane and 16-byte load
    for (int c = 8 * lane; c < R; c += 512) {
      const u32x4 x = *reinterpret_cast<const u32x4*>(dzp + c), y = *reinterpret_cast<const u32x4*>(zp + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s = __builtin_fmaf(__uint_as_float(x[e] << 16), __uint_as_float(y[e] << 16), s);
        s = __builtin_fmaf(__uint_as_float(x[e] & 0xffff0000u), __uint_as_float(y[e] & 0xffff0000u), s);
      }
    }
  } else {
    for (int c = lane; c < R; c += 64) s = __builtin_fmaf(bf2f(dzp[c]), bf2f(zp[c]), s);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) delta[((int64_t)b * 16 + h) * Lq + i] = s;
}

// Sum of the per-split dk / dv / dq partials (fixed order): out[n] = sum_s part[s][n], n < count; out is fp32, or
// bf16 (round to nearest even) with out_bf16.
__global__ __launch_bounds__(256) void khop_split_sum_kernel(const float* part, int64_t split_stride, int splits,
                                                              int64_t count, float* out, bool out_bf16) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= count) return;
  float s = part[n];
  for (int p = 1; p < splits; ++p) s += part[p * split_stride + n];
  kh_store1(out, n, s, out_bf16);
}

// The same over 4 consecutive floats per thread (count and split_stride multiples of 4, 16-byte aligned buffers),
// every split's load in flight before the adds, which keep the split order: bitwise the scalar kernel's result.
__global__ __launch_bounds__(256) void khop_split_sum4_kernel(const float* part, int64_t split_stride, int splits,
                                                               int64_t count, float* out, bool out_bf16) {
  const int64_t n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (n >= count) return;
  floatx4 s = *reinterpret_cast<const floatx4*>(part + n);
  int p = 1;
  for (; p + 8 <= splits; p += 8) {
    floatx4 x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = *reinterpret_cast<const floatx4*>(part + (int64_t)(p + u) * split_stride + n);
#pragma unroll
    for (int u = 0; u < 8; ++u) s += x[u];
  }
  for (; p < splits; ++p) s += *reinterpret_cast<const floatx4*>(part + (int64_t)p * split_stride + n);
  kh_store4(out, n, s, out_bf16);
}

inline bool kh_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// out = the fixed-order sum of `splits` partials of `count` floats at `split_stride` (one launch)
inline void kh_split_sum(const float* part, int64_t split_stride, int splits, int64_t count, float* out,
                         bool out_bf16, hipStream_t st) {
  if (count % 4 == 0 && split_stride % 4 == 0 && kh_aligned16(part) && kh_aligned16(out))
    hipLaunchKernelGGL(khop_split_sum4_kernel, dim3((unsigned)((count / 4 + 255) / 256)), dim3(256), 0, st, part,
                       split_stride, splits, count, out, out_bf16);
  else
    hipLaunchKernelGGL(khop_split_sum_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, st, part,
                       split_stride, splits, count, out, out_bf16);
}

// Key ranges of the multi-query dq kernel: 1 when the B * ceil(Lq / 4) token groups fill the GPU, else enough
// ranges for about 512 workgroups, at least 4 key tiles (128 keys) each and at most 64.
inline int kh_dq_splits(int B, int Lq, int N) {
  const int64_t groups = (int64_t)B * ((Lq + 3) / 4);
  if (groups >= 128) return 1;
  const int by_tiles = max(1, (N + 31) / 32 / 4);
  return (int)max((int64_t)1, min(min((int64_t)64, (512 + groups - 1) / groups), (int64_t)by_tiles));
}

int kh_check(const void* q, int64_t q_sb, int64_t q_si, int64_t q_sh, const void* k, int64_t k_sb, int64_t k_sn,
             const void* v, int64_t v_sb, int64_t v_sn, int B, int Lq, int N, int R, int heads, bool forward = false) {
  HLA_REQUIRE(B >= 1 && B <= 65535 && Lq >= 0 && N >= 1, HLA_S6_EINVAL, "khop: bad sizes B=%d Lq=%d N=%d", B, Lq,
              N);
  HLA_REQUIRE(heads == 16, HLA_S6_EUNSUPPORTED, "khop: %d query heads (16 supported)", heads);
  HLA_REQUIRE(R == 128 || R == 256 || R == 512 || (forward && R == 1024), HLA_S6_EUNSUPPORTED,
              "khop: latent width %d not in {128, 256, 512}%s", R, forward ? " (or 1024 forward)" : "");
  HLA_REQUIRE(q && k && v, HLA_S6_EINVAL, "khop: null input");
  HLA_REQUIRE(kh_aligned16(q) && kh_aligned16(k) && kh_aligned16(v) && q_sb % 8 == 0 && q_si % 8 == 0 &&
                  q_sh % 8 == 0 && k_sb % 8 == 0 && k_sn % 8 == 0 && v_sb % 8 == 0 && v_sn % 8 == 0,
              HLA_S6_EINVAL, "khop: q/k/v rows must be 16-byte aligned with a unit last stride");
  return HLA_S6_OK;
}

}  // namespace
}  // namespace hla

#define HLA_KH_DISPATCH(KERNEL, R, GRID, P, ST)                                                  \
  do {                                                                                           \
    switch (R) {                                                                                 \
      case 128: hipLaunchKernelGGL(KERNEL<128>, GRID, dim3(kKhThreads), 0, ST, P); break;        \
      case 256: hipLaunchKernelGGL(KERNEL<256>, GRID, dim3(kKhThreads), 0, ST, P); break;        \
      default: hipLaunchKernelGGL(KERNEL<512>, GRID, dim3(kKhThreads), 0, ST, P); break;         \
    }                                                                                            \
  } while (0)

extern "C" int hla_s6_khop_bounds(const uint8_t* mask, int64_t m_sb, int64_t m_si, int32_t B, int32_t Lq, int32_t N,
                                  int32_t* bound, void* stream) {
  using namespace hla;
  HLA_REQUIRE(B >= 1 && Lq >= 0 && N >= 1 && bound, HLA_S6_EINVAL, "khop_bounds: bad arguments");
  const int64_t rows = (int64_t)B * Lq;
  if (rows == 0) return HLA_S6_OK;
  hipLaunchKernelGGL(khop_bound_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, as_stream(stream), mask,
                     m_sb, m_si, B, Lq, N, bound);
  return check_launch("khop_bounds");
}

extern "C" int hla_s6_khop_forward(const void* q, int64_t q_sb, int64_t q_si, int64_t q_sh, const void* k,
                                   int64_t k_sb, int64_t k_sn, const void* v, int64_t v_sb, int64_t v_sn,
                                   const uint8_t* mask, int64_t m_sb, int64_t m_si, const int32_t* bound, int32_t B,
                                   int32_t Lq, int32_t N, int32_t heads, int32_t width, float scale, void* z,
                                   int64_t z_sb, int64_t z_si, int64_t z_sh, float* lse, void* stream) {
  using namespace hla;
  int rc = kh_check(q, q_sb, q_si, q_sh, k, k_sb, k_sn, v, v_sb, v_sn, B, Lq, N, width, heads, true);
  if (rc != HLA_S6_OK) return rc;
  if (Lq == 0) return HLA_S6_OK;
  HLA_REQUIRE(bound && z && lse, HLA_S6_EINVAL, "khop_forward: null bound / output");
  const bool linear = q_sb == (int64_t)Lq * q_si && z_sb == (int64_t)Lq * z_si && k_sn == v_sn &&
                      k_sb == (int64_t)N * k_sn && v_sb == (int64_t)N * v_sn;
  HLA_REQUIRE(width != 1024 || (linear && N % 16 == 0), HLA_S6_EUNSUPPORTED,
              "khop_forward: width 1024 needs token-linear q / z rows, contiguous k / v and N a multiple of 16");
  // rows linear in the token index (t = b * Lq + i): the multi-query history kernel of the serving path runs it
  if (linear) {
    rc = khop_forward_mq(q, q_si, q_sh, k, v, k_sn, B, Lq, N, width, mask, m_sb, m_si, bound, scale, z, z_si, z_sh,
                         lse, as_stream(stream));
    if (rc != HLA_S6_EUNSUPPORTED) return rc;
  }
  HLA_REQUIRE(width != 1024, HLA_S6_EUNSUPPORTED, "khop_forward: width 1024 runs on the multi-query form only");
  KhopParams p = {};
  p.q = static_cast<const uint16_t*>(q);
  p.q_sb = q_sb; p.q_si = q_si; p.q_sh = q_sh;
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.k_sb = k_sb; p.k_sn = k_sn; p.v_sb = v_sb; p.v_sn = v_sn;
  p.mask = mask; p.m_sb = m_sb; p.m_si = m_si;
  p.bound = bound;
  p.B = B; p.Lq = Lq; p.N = N;
  p.scale = scale;
  p.scale_log2 = scale * kLog2e;
  p.z = static_cast<uint16_t*>(z);
  p.z_sb = z_sb; p.z_si = z_si; p.z_sh = z_sh;
  p.lse = lse;
  const dim3 grid((unsigned)((Lq + 1) / 2), (unsigned)B);
  HLA_KH_DISPATCH(khop_fwd, width, grid, p, as_stream(stream));
  return check_launch("khop_forward");
}

extern "C" int64_t hla_s6_khop_backward_workspace(int32_t B, int32_t Lq, int32_t N, int32_t width,
                                                   int32_t key_splits) {
  using namespace hla;
  if (B < 1 || Lq < 0 || N < 1 || width < 1 || key_splits < 1) return 0;
  const int64_t kv = key_splits > 1 ? 2 * (int64_t)key_splits * B * N * width : 0;
  const int qs = (width == 512 || width == 256) && N % 16 == 0 && Lq > 0 ? kh_dq_splits(B, Lq, N) : 1;
  const int64_t dqp = qs > 1 ? (int64_t)qs * B * Lq * 16 * width : 0;
  return max(kv, dqp);
}

extern "C" int hla_s6_khop_backward(const void* q, int64_t q_sb, int64_t q_si, int64_t q_sh, const void* k,
                                    int64_t k_sb, int64_t k_sn, const void* v, int64_t v_sb, int64_t v_sn,
                                    const uint8_t* mask, int64_t m_sb, int64_t m_si, const int32_t* bound, int32_t B,
                                    int32_t Lq, int32_t N, int32_t heads, int32_t width, float scale, const void* z,
                                    int64_t z_sb, int64_t z_si, int64_t z_sh, const float* lse, const void* dz,
                                    int64_t dz_sb, int64_t dz_si, int64_t dz_sh, const float* dlse, float* delta,
                                    float* dq, int64_t dq_sb, int64_t dq_si, int64_t dq_sh, float* dk, int64_t dk_sb,
                                    int64_t dk_sn, float* dv, int64_t dv_sb, int64_t dv_sn, int32_t key_splits,
                                    float* workspace, int64_t workspace_floats, int32_t grads_bf16, void* stream) {
  using namespace hla;
  int rc = kh_check(q, q_sb, q_si, q_sh, k, k_sb, k_sn, v, v_sb, v_sn, B, Lq, N, width, heads);
  if (rc != HLA_S6_OK) return rc;
  HLA_REQUIRE(bound && z && lse && dz && delta, HLA_S6_EINVAL, "khop_backward: null input");
  HLA_REQUIRE(key_splits >= 1 && key_splits <= 64, HLA_S6_EINVAL, "khop_backward: key_splits %d not in [1, 64]",
              key_splits);
  HLA_REQUIRE(kh_aligned16(dz) && dz_sb % 8 == 0 && dz_si % 8 == 0 && dz_sh % 8 == 0, HLA_S6_EINVAL,
              "khop_backward: dz rows must be 16-byte aligned with a unit last stride");
  const bool need_q = dq != nullptr, need_kv = dk != nullptr || dv != nullptr;
  HLA_REQUIRE(!need_kv || (dk && dv), HLA_S6_EINVAL, "khop_backward: dk and dv come together");
  const int64_t part = (int64_t)B * N * width;  // floats of one dk (or dv) partial
  if (need_kv && key_splits > 1) {
    HLA_REQUIRE(workspace && workspace_floats >= 2 * key_splits * part, HLA_S6_EWORKSPACE,
                "khop_backward: %d key splits need a workspace of %lld floats (got %lld)", key_splits,
                (long long)(2 * key_splits * part), (long long)workspace_floats);
  }
  hipStream_t st = as_stream(stream);
  KhopParams p = {};
  p.q = static_cast<const uint16_t*>(q);
  p.q_sb = q_sb; p.q_si = q_si; p.q_sh = q_sh;
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.k_sb = k_sb; p.k_sn = k_sn; p.v_sb = v_sb; p.v_sn = v_sn;
  p.mask = mask; p.m_sb = m_sb; p.m_si = m_si;
  p.bound = bound;
  p.B = B; p.Lq = Lq; p.N = N;
  p.scale = scale;
  p.scale_log2 = scale * kLog2e;
  p.lse = const_cast<float*>(lse);
  p.dz = static_cast<const uint16_t*>(dz);
  p.dz_sb = dz_sb; p.dz_si = dz_si; p.dz_sh = dz_sh;
  p.dlse = dlse;
  p.delta = delta;
  if (Lq > 0) {
    const int64_t rows = (int64_t)B * Lq * 16;
    hipLaunchKernelGGL(khop_delta_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st,
                       static_cast<const uint16_t*>(dz), dz_sb, dz_si, dz_sh, static_cast<const uint16_t*>(z), z_sb,
                       z_si, z_sh, B, Lq, width, delta);
    if ((rc = check_launch("khop_delta")) != HLA_S6_OK) return rc;
  }
  if (need_q && Lq > 0) {
    p.dq = dq;
    p.dq_sb = dq_sb; p.dq_si = dq_si; p.dq_sh = dq_sh;
    // the multi-query form: widths 512 / 256, whole 16-key groups, 16-byte aligned fp32 dq rows and mask rows
    const bool dq4 = (width == 512 || width == 256) && N % 16 == 0 && kh_aligned16(dq) &&
                     dq_sb % 4 == 0 && dq_si % 4 == 0 && dq_sh % 4 == 0 &&
                     (!mask || (kh_aligned16(mask) && m_sb % 16 == 0 && m_si % 16 == 0));
    if (dq4) {
      // few token groups (a single query per row): key ranges with fp32 partials in the workspace, summed in a
      // fixed order into a contiguous dq
      const int64_t part_q = (int64_t)B * Lq * 16 * width;
      int qs = kh_dq_splits(B, Lq, N);
      if (qs > 1 && !(workspace && kh_aligned16(workspace) && workspace_floats >= qs * part_q &&
                      dq_sb == (int64_t)Lq * 16 * width && dq_si == 16 * width && dq_sh == width))
        qs = 1;
      if (qs > 1) {
        p.dq = workspace;
        p.dq_ss = part_q;
      }
      p.dq_bf16 = grads_bf16 != 0 && qs == 1;
      const dim3 grid4((unsigned)((Lq + 3) / 4), (unsigned)B, (unsigned)qs);
      if (width == 512 && mask) hipLaunchKernelGGL((khop_dq4<512, true>), grid4, dim3(kKhThreads), 0, st, p);
      else if (width == 512) hipLaunchKernelGGL((khop_dq4<512, false>), grid4, dim3(kKhThreads), 0, st, p);
      else if (mask) hipLaunchKernelGGL((khop_dq4<256, true>), grid4, dim3(kKhThreads), 0, st, p);
      else hipLaunchKernelGGL((khop_dq4<256, false>), grid4, dim3(kKhThreads), 0, st, p);
      if (qs > 1) {
        if ((rc = check_launch("khop_dq")) != HLA_S6_OK) return rc;
        kh_split_sum(workspace, part_q, qs, part_q, dq, grads_bf16 != 0, st);
      }
    } else {
      const dim3 grid((unsigned)((Lq + 1) / 2), (unsigned)B);
      p.dq_bf16 = grads_bf16 != 0;
      HLA_KH_DISPATCH(khop_dq, width, grid, p, st);
    }
    if ((rc = check_launch("khop_dq")) != HLA_S6_OK) return rc;
  }
  if (need_kv) {
    const bool split = key_splits > 1;
    HLA_REQUIRE(!split || (dk_sb == (int64_t)N * width && dk_sn == width && dv_sb == (int64_t)N * width &&
                           dv_sn == width),
                HLA_S6_EINVAL, "khop_backward: with key splits dk / dv must be contiguous [B, N, width]");
    p.key_splits = key_splits;
    p.kv_bf16 = grads_bf16 != 0 && !split;
    p.dk = split ? workspace : dk;
    p.dv = split ? workspace + key_splits * part : dv;
    p.dk_sb = split ? (int64_t)N * width : dk_sb;
    p.dk_sn = split ? width : dk_sn;
    p.dv_sb = split ? (int64_t)N * width : dv_sb;
    p.dv_sn = split ? width : dv_sn;
    p.dk_ss = p.dv_ss = part;
    // the multi-query form: widths 512 / 256, whole 16-key groups, 16-byte aligned fp32 dk / dv rows and mask rows
    const bool kv4 = (width == 512 || width == 256) && N % 16 == 0 && kh_aligned16(p.dk) &&
                     kh_aligned16(p.dv) && p.dk_sb % 4 == 0 && p.dk_sn % 4 == 0 && p.dv_sb % 4 == 0 &&
                     p.dv_sn % 4 == 0 && (!mask || (kh_aligned16(mask) && m_sb % 16 == 0 && m_si % 16 == 0));
    if (kv4) {
      const dim3 grid4((unsigned)((N + 63) / 64), (unsigned)B, (unsigned)key_splits);
      if (width == 512 && mask) hipLaunchKernelGGL((khop_dkdv4<512, true>), grid4, dim3(kKhThreads), 0, st, p);
      else if (width == 512) hipLaunchKernelGGL((khop_dkdv4<512, false>), grid4, dim3(kKhThreads), 0, st, p);
      else if (mask) hipLaunchKernelGGL((khop_dkdv4<256, true>), grid4, dim3(kKhThreads), 0, st, p);
      else hipLaunchKernelGGL((khop_dkdv4<256, false>), grid4, dim3(kKhThreads), 0, st, p);
    } else {
      const dim3 grid((unsigned)((N + kKhKeys - 1) / kKhKeys), (unsigned)B, (unsigned)key_splits);
      HLA_KH_DISPATCH(khop_dkdv, width, grid, p, st);
    }
    if ((rc = check_launch("khop_dkdv")) != HLA_S6_OK) return rc;
    if (split) {
      kh_split_sum(workspace, part, key_splits, part, dk, grads_bf16 != 0, st);
      kh_split_sum(workspace + key_splits * part, part, key_splits, part, dv, grads_bf16 != 0, st);
      if ((rc = check_launch("khop_split_sum")) != HLA_S6_OK) return rc;
    }
  }
  return HLA_S6_OK;
}
