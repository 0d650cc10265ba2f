// Multi-query latent history attention on contiguous rows with an arbitrary visibility mask, in fp32 arithmetic:
// the reference's default precision of the K-hop replay / training op (hla/latent/history_gemm.py:19-24,37,46-66,
// precision 'fp32': IEEE fp32 GEMMs; the same arithmetic as its fp32 CUDA-core 'triton' backend,
// hla/latent/fused_history.py:126-153, and its dense 'reference' backend).
//
//   q [B, Lq, 16, R], k/v [B, N, R] fp32 (rows shared by the 16 heads), mask [B, Lq, N] (nonzero = visible)
//   z[b,i,h] = softmax_j(scale q.k_j | visible) . v,  lse[b,h,i] (natural log; -inf and z = 0 with no visible key)
//   backward (P = exp(s - lse), delta = dz.z):  dv = P^T dz,  dS = P (dz.v - delta + dlse) scale,
//                                               dq = dS k,    dk = dS^T q
//
// Every product runs on v_mfma_f32_16x16x4_f32 (fp32 operands, fp32 accumulation). A wave owns RC latent columns
// of one token (forward, dq) or of one 16-key block (dk / dv); the R / RC waves that share a token (key block) sum
// their partial 16 x 16 score blocks through LDS in a fixed order, so each of them forms the same P. The operand
// tiles of 16 rows x R (K and V, or Q and dZ) are staged in LDS (rows padded by 4 floats) from registers loaded one
// step ahead. Products over the latent columns take both operands as 16-byte LDS reads (column c of k-step t is
// 4 (l / 16) + t within a 16-column chunk, the same for both operands); products over keys or heads take the
// row-major tile as 16-byte reads too, by giving output row m of column block cb the column 4 m + cb, so the four
// blocks of a lane's 16-byte read are four MFMAs and a lane's results are 16 consecutive columns.
//
// Each token's key bound (1 + its last visible key, from the mask) limits the key range, so a causal mask costs
// half the work without a causality promise.
#include "common.h"

namespace hla {
namespace {

constexpr int kFKeys = 16;  // keys (forward, dq) or query heads (dk / dv) per step

__device__ __forceinline__ floatx4 mfma_f32(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct KfParams {
  const float* q;
  int64_t q_sb, q_si, q_sh;
  const float* k;
  const float* v;
  int64_t k_sb, k_sn, v_sb, v_sn;
  const uint8_t* mask;  // may be null (then every key below the bound is visible)
  int64_t m_sb, m_si;
  const int32_t* bound;  // [B * Lq]
  int B, Lq, N;
  float scale, scale_log2;
  float* z;
  int64_t z_sb, z_si, z_sh;
  float* lse;  // [B, 16, Lq]
  const float* dz;
  int64_t dz_sb, dz_si, dz_sh;
  const float* dlse;   // [B, 16, Lq] or null
  const float* delta;  // [B, 16, Lq]
  float* dq;
  int64_t dq_sb, dq_si, dq_sh;
  float* dk;
  float* dv;
  int64_t dk_sb, dk_sn, dv_sb, dv_sn;
  int key_splits;      // dk / dv: token ranges per key block; range s writes its partial at dk + s * kv_ss
  int64_t kv_ss;
};

// Geometry of a kernel over width R with RC columns per wave and W waves: CS waves per token (key block), G tokens
// (key blocks) per workgroup.
template <int R, int RC, int W>
struct KfGeo {
  static constexpr int THREADS = 64 * W;
  static constexpr int CS = R / RC;
  static constexpr int G = W / CS;
  static constexpr int NC = RC / 16;   // 16-column chunks of a wave (products over the columns)
  static constexpr int NB = RC / 64;   // 64-column blocks of a wave (products over keys / heads)
  static constexpr int RS = R + 4;     // LDS row stride of a tile, floats
  static constexpr int TL = kFKeys * R / 4 / THREADS;  // 16-byte pieces per thread per tile
  // the score and dP exchanges share one LDS buffer (one more barrier) when two would not fit beside the tiles
  static constexpr bool ONE_X = 2 * kFKeys * RS * 4 + 2 * W * 64 * 16 > 160 * 1024;
  static_assert(CS >= 1 && CS <= W && W % CS == 0 && NB >= 1 && TL >= 1, "unsupported width / column split");
};

// A compiler-only fence: LDS operand reads are not hoisted across it (each 16-byte read feeds four 32-cycle MFMAs, so
// reads two steps ahead keep the matrix pipe fed; hoisting all of them would cost registers the kernels lack).
__device__ __forceinline__ void kf_fence() { asm volatile("" ::: "memory"); }

template <int R, int RC, int W>
using KfRegs = floatx4[KfGeo<R, RC, W>::TL];   // one tile's share of a thread
template <int R, int RC, int W>
using KfAcc = floatx4[KfGeo<R, RC, W>::NB][4];  // a wave's 16 x RC accumulator (see kf_rows)
template <int R, int RC, int W>
using KfCols = floatx4[KfGeo<R, RC, W>::NC];   // a lane's B operand over the wave's columns (see kf_cols)

// 16 rows x R of a row-major fp32 matrix into registers (piece p = it * THREADS + tid is row p / (R / 4), columns
// 4 (p % (R / 4)) .. +4); rowp(r) is an in-bounds row pointer.
template <int R, int RC, int W, class RowP>
__device__ __forceinline__ void kf_load(KfRegs<R, RC, W>& reg, RowP rowp) {
#pragma unroll
  for (int it = 0; it < KfGeo<R, RC, W>::TL; ++it) {
    const int p = it * KfGeo<R, RC, W>::THREADS + threadIdx.x;
    reg[it] = *reinterpret_cast<const floatx4*>(rowp(p / (R / 4)) + 4 * (p % (R / 4)));
  }
}

template <int R, int RC, int W>
__device__ __forceinline__ void kf_store(float* tile, const KfRegs<R, RC, W>& reg) {
#pragma unroll
  for (int it = 0; it < KfGeo<R, RC, W>::TL; ++it) {
    const int p = it * KfGeo<R, RC, W>::THREADS + threadIdx.x;
    *reinterpret_cast<floatx4*>(tile + (p / (R / 4)) * KfGeo<R, RC, W>::RS + 4 * (p % (R / 4))) = reg[it];
  }
}

// Partial D[m][n] = sum over the wave's columns [c0, c0 + RC) of A[m][c] B[n][c], with A's 16 rows a row-major LDS
// tile and B held by the lane as breg[c][t] = B[l % 16][c0 + 16 c + 4 (l / 16) + t]. Lane l gets D[4 (l / 16) + i]
// [l % 16] in element i.
template <int R, int RC, int W>
__device__ __forceinline__ floatx4 kf_cols(const float* tile, int c0, const KfCols<R, RC, W>& breg) {
  const int lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
  const float* ap = tile + l16 * KfGeo<R, RC, W>::RS + c0 + 4 * g;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < KfGeo<R, RC, W>::NC; ++c) {
    const floatx4 a = *reinterpret_cast<const floatx4*>(ap + 16 * c);
#pragma unroll
    for (int t = 0; t < 4; ++t) acc = mfma_f32(a[t], breg[c][t], acc);
    if (c % 2 == 1) kf_fence();
  }
  return acc;
}

// acc[nb][cb] += T^T . W over the 16 rows of a row-major LDS tile T (row r = 4 (l / 16) + st holds the lane's
// weight w[st] for its output column l % 16): output row m of block (nb, cb) is column c0 + 64 nb + 4 m + cb.
template <int R, int RC, int W>
__device__ __forceinline__ void kf_rows(KfAcc<R, RC, W>& acc, const float* tile, int c0, const floatx4& w) {
  const int lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const float* rp = tile + (4 * g + st) * KfGeo<R, RC, W>::RS + c0 + 4 * l16;
#pragma unroll
    for (int nb = 0; nb < KfGeo<R, RC, W>::NB; ++nb) {
      const floatx4 a = *reinterpret_cast<const floatx4*>(rp + 64 * nb);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) acc[nb][cb] = mfma_f32(a[cb], w[st], acc[nb][cb]);
    }
    if (st % 2 == 1) kf_fence();
  }
}

// Store of a kf_rows accumulator scaled by s: the lane's 16 columns c0 + 64 nb + 16 (l / 16) + 4 i + cb of row ptr.
template <int R, int RC, int W>
__device__ __forceinline__ void kf_store_rows(float* row, int c0, const KfAcc<R, RC, W>& acc, float s) {
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int nb = 0; nb < KfGeo<R, RC, W>::NB; ++nb)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<floatx4*>(row + c0 + 64 * nb + 16 * g + 4 * i) =
          floatx4{acc[nb][0][i] * s, acc[nb][1][i] * s, acc[nb][2][i] * s, acc[nb][3][i] * s};
}

// Sum of the CS partial blocks of this wave's token (key block) through LDS, in a fixed order.
template <int CS>
__device__ __forceinline__ floatx4 kf_exchange(floatx4 part, floatx4 (*xs)[64], int wave, int first) {
  if (CS == 1) return part;
  const int lane = threadIdx.x & 63;
  xs[wave][lane] = part;
  __syncthreads();
  floatx4 s = xs[first][lane];
#pragma unroll
  for (int c = 1; c < CS; ++c) s += xs[first + c][lane];
  return s;
}

// The four mask bytes of keys key0 .. key0 + 3 for query row `row` (a row pointer), 1 without a mask.
__device__ __forceinline__ void kf_mask4(const uint8_t* row, int key0, int N, uint8_t (&m)[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) m[e] = row ? row[min(key0 + e, N - 1)] : (uint8_t)1;
}

// Direct global -> LDS copy of a 16-row tile (rowp(r) an in-bounds row pointer, R floats per row) into a padded LDS
// tile at LDS byte address `tile`: 1 KB per wave instruction, the workgroup's waves taking the rows in turn. Every
// address is wave-uniform and kept in scalar registers (the wave index is read through readfirstlane). The copies
// are not counted by the compiler: the caller waits with kf_wait_copies() before the barrier after which the tile
// is read.
template <int R, int RC, int W, class RowP>
__device__ __forceinline__ void kf_copy_tile(uint32_t tile, RowP rowp) {
  constexpr int PER_ROW = R / 256;
  constexpr int PER_WAVE = kFKeys * PER_ROW / W;
  static_assert(PER_ROW >= 1 && PER_WAVE >= 1 && kFKeys * PER_ROW % W == 0, "tile copy split");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane_off = 16u * (threadIdx.x & 63);
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int c = wave * PER_WAVE + i, r = c / PER_ROW, j = c % PER_ROW;
    const int64_t row = uniform64(reinterpret_cast<int64_t>(rowp(r)));
    const uint32_t dst = __builtin_amdgcn_readfirstlane(tile + (uint32_t)((r * KfGeo<R, RC, W>::RS + 256 * j) * 4));
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(dst), "v"(lane_off + 1024u * j),
                 "s"(reinterpret_cast<const void*>(row))
                 : "memory", "m0");
  }
}
// LDS byte address of a shared array
__device__ __forceinline__ uint32_t kf_lds(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}
__device__ __forceinline__ void kf_wait_copies() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---- forward: one workgroup per G consecutive tokens of a batch row (longest rows first) ------------------------
template <int R, int RC, int W>
__global__ __launch_bounds__(64 * W) void khf_fwd(KfParams a) {
  using G_ = KfGeo<R, RC, W>;
  constexpr int CS = G_::CS, TG = G_::G;
  __shared__ __attribute__((aligned(16))) float ks[kFKeys * G_::RS];
  __shared__ __attribute__((aligned(16))) float vs[kFKeys * G_::RS];
  __shared__ __attribute__((aligned(16))) floatx4 xs[CS > 1 ? W : 1][64];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  const int tok = wave / CS, c0 = (wave % CS) * RC;
  const int b = blockIdx.y;
  const int groups = (a.Lq + TG - 1) / TG;
  const int i0 = (groups - 1 - (int)blockIdx.x) * TG;
  const int ntok = min(TG, a.Lq - i0);
  const bool tok_ok = tok < ntok;
  const int ti = i0 + min(tok, ntok - 1);
  const int64_t trow = (int64_t)b * a.Lq;
  int nkeys = 0;
  for (int t = 0; t < ntok; ++t) nkeys = max(nkeys, min(a.bound[trow + i0 + t], a.N));
  const int my_bound = tok_ok ? min(a.bound[trow + ti], a.N) : 0;
  const uint8_t* mrow = a.mask ? a.mask + (int64_t)b * a.m_sb + (int64_t)ti * a.m_si : nullptr;

  floatx4 qv[G_::NC];
  {
    const float* qp = a.q + (int64_t)b * a.q_sb + (int64_t)ti * a.q_si + (int64_t)l16 * a.q_sh + c0 + 4 * g;
#pragma unroll
    for (int c = 0; c < G_::NC; ++c) qv[c] = *reinterpret_cast<const floatx4*>(qp + 16 * c);
  }
  floatx4 acc[G_::NB][4];
#pragma unroll
  for (int nb = 0; nb < G_::NB; ++nb)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[nb][cb] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_part = 0.f;

  floatx4 kr[G_::TL], vr[G_::TL];
  uint8_t m_next[4] = {1, 1, 1, 1}, m_cur[4];
  auto load = [&](int kt) {
    kf_load<R, RC, W>(kr, [&](int r) { return a.k + (int64_t)b * a.k_sb + (int64_t)min(kt + r, a.N - 1) * a.k_sn; });
    kf_load<R, RC, W>(vr, [&](int r) { return a.v + (int64_t)b * a.v_sb + (int64_t)min(kt + r, a.N - 1) * a.v_sn; });
    kf_mask4(mrow, kt + 4 * g, a.N, m_next);
  };
  if (nkeys > 0) load(0);
  for (int kt = 0; kt < nkeys; kt += kFKeys) {
    __syncthreads();  // the previous tile's readers are done
    kf_store<R, RC, W>(ks, kr);
    kf_store<R, RC, W>(vs, vr);
#pragma unroll
    for (int e = 0; e < 4; ++e) m_cur[e] = m_next[e];
    __syncthreads();
    if (kt + kFKeys < nkeys) load(kt + kFKeys);
    // S^T[key 4 g + i][head l16]
    const floatx4 s = kf_exchange<CS>(kf_cols<R, RC, W>(ks, c0, qv), xs, wave, tok * CS);
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kt + 4 * g + i;
      x[i] = tok_ok && key < my_bound && m_cur[i] ? s[i] * a.scale_log2 : -INFINITY;
    }
    const float mx = wave_max16x4(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);  // 0 while m_run = -inf
    floatx4 p;
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = fast_exp2(x[i] - m_use);
    l_part = l_part * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    m_run = m_new;
#pragma unroll
    for (int nb = 0; nb < G_::NB; ++nb)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) acc[nb][cb] *= alpha;
    kf_rows<R, RC, W>(acc, vs, c0, p);  // O^T += V^T P^T
  }
  const float l = wave_sum16x4(l_part);
  if (tok_ok) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    kf_store_rows<R, RC, W>(a.z + (int64_t)b * a.z_sb + (int64_t)ti * a.z_si + (int64_t)l16 * a.z_sh, c0, acc, inv);
    if (g == 0 && c0 == 0)
      a.lse[((int64_t)b * 16 + l16) * a.Lq + ti] = l > 0.f ? (m_run + log2f(l)) * kLn2 : -INFINITY;
  }
}

// ---- dq: the forward's layout; per key tile S and dP, then dQ^T += K^T dS^T ------------------------------------
template <int R, int RC, int W>
__global__ __launch_bounds__(64 * W) void khf_dq(KfParams a) {
  using G_ = KfGeo<R, RC, W>;
  constexpr int CS = G_::CS, TG = G_::G;
  // width 1024: the V tile goes global -> LDS directly (the registers of a second staged tile do not fit)
  constexpr bool DMA = R >= 1024;
  __shared__ __attribute__((aligned(16))) float ks[kFKeys * G_::RS];
  __shared__ __attribute__((aligned(16))) float vs[kFKeys * G_::RS];
  __shared__ __attribute__((aligned(16))) floatx4 xs[CS > 1 ? W : 1][64];
  __shared__ __attribute__((aligned(16))) floatx4 xd[CS > 1 && !G_::ONE_X ? W : 1][64];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  const int tok = wave / CS, c0 = (wave % CS) * RC;
  const int b = blockIdx.y;
  const int groups = (a.Lq + TG - 1) / TG;
  const int i0 = (groups - 1 - (int)blockIdx.x) * TG;
  const int ntok = min(TG, a.Lq - i0);
  const bool tok_ok = tok < ntok;
  const int ti = i0 + min(tok, ntok - 1);
  const int64_t trow = (int64_t)b * a.Lq;
  int nkeys = 0;
  for (int t = 0; t < ntok; ++t) nkeys = max(nkeys, min(a.bound[trow + i0 + t], a.N));
  const int my_bound = tok_ok ? min(a.bound[trow + ti], a.N) : 0;
  const uint8_t* mrow = a.mask ? a.mask + (int64_t)b * a.m_sb + (int64_t)ti * a.m_si : nullptr;
  // row constants of head l16: lse in the log2 domain (0 without history: its P are all 0) and delta - dlse
  const int64_t ridx = ((int64_t)b * 16 + l16) * a.Lq + ti;
  const float lse_n = a.lse[ridx];
  const bool empty = !(lse_n > -INFINITY);
  const float lse2 = empty ? 0.f : lse_n * kLog2e;
  const float dd = a.delta[ridx] - (empty || !a.dlse ? 0.f : a.dlse[ridx]);

  floatx4 qv[G_::NC], dzv[G_::NC];
  {
    const float* qp = a.q + (int64_t)b * a.q_sb + (int64_t)ti * a.q_si + (int64_t)l16 * a.q_sh + c0 + 4 * g;
    const float* dp = a.dz + (int64_t)b * a.dz_sb + (int64_t)ti * a.dz_si + (int64_t)l16 * a.dz_sh + c0 + 4 * g;
#pragma unroll
    for (int c = 0; c < G_::NC; ++c) {
      qv[c] = *reinterpret_cast<const floatx4*>(qp + 16 * c);
      dzv[c] = *reinterpret_cast<const floatx4*>(dp + 16 * c);
    }
  }
  floatx4 acc[G_::NB][4];
#pragma unroll
  for (int nb = 0; nb < G_::NB; ++nb)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[nb][cb] = floatx4{0.f, 0.f, 0.f, 0.f};

  floatx4 kr[G_::TL], vr[G_::TL];
  uint8_t m_next[4] = {1, 1, 1, 1}, m_cur[4];
  auto load = [&](int kt) {
    kf_load<R, RC, W>(kr, [&](int r) { return a.k + (int64_t)b * a.k_sb + (int64_t)min(kt + r, a.N - 1) * a.k_sn; });
    if (!DMA)
      kf_load<R, RC, W>(vr,
                        [&](int r) { return a.v + (int64_t)b * a.v_sb + (int64_t)min(kt + r, a.N - 1) * a.v_sn; });
    kf_mask4(mrow, kt + 4 * g, a.N, m_next);
  };
  if (nkeys > 0) load(0);
  for (int kt = 0; kt < nkeys; kt += kFKeys) {
    __syncthreads();
    kf_store<R, RC, W>(ks, kr);
    if constexpr (DMA)  // the V tile, read first by the dP product after the score exchange
      kf_copy_tile<R, RC, W>(kf_lds(vs), [&](int r) {
        return a.v + (int64_t)b * a.v_sb + (int64_t)min(kt + r, a.N - 1) * a.v_sn;
      });
    else
      kf_store<R, RC, W>(vs, vr);
#pragma unroll
    for (int e = 0; e < 4; ++e) m_cur[e] = m_next[e];
    __syncthreads();
    if (!DMA && kt + kFKeys < nkeys) load(kt + kFKeys);
    const floatx4 s_part = kf_cols<R, RC, W>(ks, c0, qv);
    if (DMA) kf_wait_copies();  // this wave's V copies; the exchange's barrier then publishes every wave's
    const floatx4 s = kf_exchange<CS>(s_part, xs, wave, tok * CS);
    if (DMA && kt + kFKeys < nkeys) load(kt + kFKeys);
    if (G_::ONE_X && CS > 1) __syncthreads();  // every wave has its sums before the buffer is reused
    const floatx4 dpv = kf_exchange<CS>(kf_cols<R, RC, W>(vs, c0, dzv), G_::ONE_X ? xs : xd, wave, tok * CS);
    floatx4 ds;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kt + 4 * g + i;
      const bool vis = tok_ok && key < my_bound && m_cur[i];
      const float p = vis ? fast_exp2(s[i] * a.scale_log2 - lse2) : 0.f;
      ds[i] = p * (dpv[i] - dd) * a.scale;
    }
    kf_rows<R, RC, W>(acc, ks, c0, ds);  // dQ^T += K^T dS^T
  }
  if (tok_ok)
    kf_store_rows<R, RC, W>(a.dq + (int64_t)b * a.dq_sb + (int64_t)ti * a.dq_si + (int64_t)l16 * a.dq_sh, c0, acc,
                         1.f);
}

// ---- dk / dv: one workgroup per (G blocks of 16 keys, batch row, token range); query tokens stream through LDS --
// (their 16 head rows of q and dz), per token S = Q K^T and dP = dZ V^T (16 heads x 16 keys), then
// dV^T += dZ^T P and dK^T += Q^T dS over the wave's columns.
template <int R, int RC, int W>
__global__ __launch_bounds__(64 * W) void khf_dkdv(KfParams a) {
  using G_ = KfGeo<R, RC, W>;
  constexpr int CS = G_::CS, KBW = G_::G;
  // widths 512 and 1024: the Q and dZ tiles go global -> LDS directly (their staging registers do not fit beside
  // the resident K / V operands and dK / dV accumulators)
  constexpr bool DMA = R >= 512;
  __shared__ __attribute__((aligned(16))) float qs[kFKeys * G_::RS];
  __shared__ __attribute__((aligned(16))) float zs[kFKeys * G_::RS];
  __shared__ __attribute__((aligned(16))) floatx4 xs[CS > 1 ? W : 1][64];
  __shared__ __attribute__((aligned(16))) floatx4 xd[CS > 1 && !G_::ONE_X ? W : 1][64];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  const int kb = wave / CS, c0 = (wave % CS) * RC;
  const int b = blockIdx.y;
  const int key0 = (int)blockIdx.x * (16 * KBW);
  const int key = key0 + 16 * kb + l16;  // this lane's key (columns of S)
  const bool key_ok = key < a.N;
  const int kc = min(key, a.N - 1);
  // the token range of this split
  const int split = blockIdx.z;
  const int t_lo = (int)((int64_t)a.Lq * split / a.key_splits), t_hi = (int)((int64_t)a.Lq * (split + 1) / a.key_splits);
  const int64_t trow = (int64_t)b * a.Lq;

  floatx4 kv[G_::NC], vv[G_::NC];  // K^T / V^T as B operands: lane l holds row `key`, columns c0 + 16 c + 4 g ..
  {
    const float* kp = a.k + (int64_t)b * a.k_sb + (int64_t)kc * a.k_sn + c0 + 4 * g;
    const float* vp = a.v + (int64_t)b * a.v_sb + (int64_t)kc * a.v_sn + c0 + 4 * g;
#pragma unroll
    for (int c = 0; c < G_::NC; ++c) {
      kv[c] = *reinterpret_cast<const floatx4*>(kp + 16 * c);
      vv[c] = *reinterpret_cast<const floatx4*>(vp + 16 * c);
    }
  }
  floatx4 dk_acc[G_::NB][4], dv_acc[G_::NB][4];
#pragma unroll
  for (int nb = 0; nb < G_::NB; ++nb)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) dk_acc[nb][cb] = dv_acc[nb][cb] = floatx4{0.f, 0.f, 0.f, 0.f};

  // The range's tokens that see any key of the block (bound above key0), last to first: the workgroups of a batch
  // row and range all start at the range's last token and step down together, so the token tiles they stream are
  // read about once per XCD and served to the others from L2. prev_token(t) is the highest such token below t
  // (t_lo - 1 if none), found 64 tokens per probe.
  auto prev_token = [&](int t) {
    while (t > t_lo) {
      const int base = max(t_lo, t - 64);
      const bool seen = base + lane < t && a.bound[trow + base + lane] > key0;
      const uint64_t m = __ballot(seen);
      if (m) return base + 63 - __clzll(m);
      t = base;
    }
    return t_lo - 1;
  };
  float c_lse[4], c_dd[4], n_lse[4], n_dd[4];  // row constants of heads 4 g + i (current / next token)
  int c_bound = 0, n_bound = 0;
  uint8_t c_m = 1, n_m = 1;
  auto load_consts = [&](int t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t ridx = ((int64_t)b * 16 + 4 * g + i) * a.Lq + t;
      const float l = a.lse[ridx];
      const bool empty = !(l > -INFINITY);
      n_lse[i] = empty ? 0.f : l * kLog2e;
      n_dd[i] = a.delta[ridx] - (empty || !a.dlse ? 0.f : a.dlse[ridx]);
    }
    n_bound = min(a.bound[trow + t], a.N);
    n_m = a.mask ? a.mask[(int64_t)b * a.m_sb + (int64_t)t * a.m_si + kc] : (uint8_t)1;
  };
  auto take_consts = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c_lse[i] = n_lse[i];
      c_dd[i] = n_dd[i];
    }
    c_bound = n_bound;
    c_m = n_m;
  };
  const auto qrow = [&](int t) {
    return [&, t](int r) { return a.q + (int64_t)b * a.q_sb + (int64_t)t * a.q_si + (int64_t)r * a.q_sh; };
  };
  const auto zrow = [&](int t) {
    return [&, t](int r) { return a.dz + (int64_t)b * a.dz_sb + (int64_t)t * a.dz_si + (int64_t)r * a.dz_sh; };
  };
  // P and dS of the step from the score and dP sums (head 4 g + i, key l16)
  auto p_ds = [&](const floatx4& s, const floatx4& dpv, floatx4& p, floatx4& ds) {
    const bool vis = key_ok && key < c_bound && c_m != 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = vis ? fast_exp2(s[i] * a.scale_log2 - c_lse[i]) : 0.f;
      ds[i] = p[i] * (dpv[i] - c_dd[i]) * a.scale;
    }
  };
  int t = prev_token(t_hi);
  if constexpr (DMA) {
    // width 1024: both tiles go global -> LDS directly. dZ(t) is copied while S is computed; Q(t) is last read by
    // the dK product, which runs before dV, so Q of the next token is copied while dV is computed.
    if (t >= t_lo) {
      kf_copy_tile<R, RC, W>(kf_lds(qs), qrow(t));
      load_consts(t);
    }
    while (t >= t_lo) {
      kf_wait_copies();  // this wave's Q copies
      __syncthreads();   // Q visible to every wave; every wave is done with the previous token's dZ tile
      kf_copy_tile<R, RC, W>(kf_lds(zs), zrow(t));
      take_consts();
      const int t_next = prev_token(t);
      if (t_next >= t_lo) load_consts(t_next);
      const floatx4 s_part = kf_cols<R, RC, W>(qs, c0, kv);
      kf_wait_copies();  // this wave's dZ copies; the exchange's barrier then publishes every wave's
      const floatx4 s = kf_exchange<CS>(s_part, xs, wave, kb * CS);
      if (G_::ONE_X && CS > 1) __syncthreads();
      const floatx4 dpv = kf_exchange<CS>(kf_cols<R, RC, W>(zs, c0, vv), G_::ONE_X ? xs : xd, wave, kb * CS);
      floatx4 p, ds;
      p_ds(s, dpv, p, ds);
      kf_rows<R, RC, W>(dk_acc, qs, c0, ds);  // dK^T += Q^T dS
      __syncthreads();                         // every wave is done with the Q tile
      if (t_next >= t_lo) kf_copy_tile<R, RC, W>(kf_lds(qs), qrow(t_next));
      kf_rows<R, RC, W>(dv_acc, zs, c0, p);   // dV^T += dZ^T P
      t = t_next;
    }
  } else {
    floatx4 qr[G_::TL], zr[G_::TL];
    auto load = [&](int t) {
      kf_load<R, RC, W>(qr, qrow(t));
      kf_load<R, RC, W>(zr, zrow(t));
      load_consts(t);
    };
    if (t >= t_lo) load(t);
    while (t >= t_lo) {
      __syncthreads();
      kf_store<R, RC, W>(qs, qr);
      kf_store<R, RC, W>(zs, zr);
      take_consts();
      __syncthreads();
      const int t_next = prev_token(t);
      if (t_next >= t_lo) load(t_next);
      // S[head 4 g + i][key l16], dP likewise
      const floatx4 s = kf_exchange<CS>(kf_cols<R, RC, W>(qs, c0, kv), xs, wave, kb * CS);
      if (G_::ONE_X && CS > 1) __syncthreads();  // every wave has its sums before the buffer is reused
      const floatx4 dpv = kf_exchange<CS>(kf_cols<R, RC, W>(zs, c0, vv), G_::ONE_X ? xs : xd, wave, kb * CS);
      floatx4 p, ds;
      p_ds(s, dpv, p, ds);
      kf_rows<R, RC, W>(dv_acc, zs, c0, p);   // dV^T += dZ^T P
      kf_rows<R, RC, W>(dk_acc, qs, c0, ds);  // dK^T += Q^T dS
      t = t_next;
    }
  }
  if (key_ok) {
    const int64_t off = a.key_splits > 1 ? (int64_t)split * a.kv_ss : 0;
    kf_store_rows<R, RC, W>(a.dv + off + (int64_t)b * a.dv_sb + (int64_t)key * a.dv_sn, c0, dv_acc, 1.f);
    kf_store_rows<R, RC, W>(a.dk + off + (int64_t)b * a.dk_sb + (int64_t)key * a.dk_sn, c0, dk_acc, 1.f);
  }
}

// delta[b, h, i] = sum_c dz[b, i, h, c] * z[b, i, h, c] (fp32). One wave per row.
__global__ __launch_bounds__(256) void khf_delta_kernel(const float* dz, int64_t dz_sb, int64_t dz_si, int64_t dz_sh,
                                                        const float* z, int64_t z_sb, int64_t z_si, int64_t z_sh,
                                                        int B, int Lq, int R, float* delta) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= (int64_t)B * Lq * 16) return;
  const int h = (int)(row % 16);
  const int64_t t = row / 16;
  const int b = (int)(t / Lq), i = (int)(t % Lq);
  const float* dzp = dz + b * dz_sb + i * dz_si + h * dz_sh;
  const float* zp = z + b * z_sb + i * z_si + h * z_sh;
  float s = 0.f;
  for (int c = 4 * lane; c < R; c += 256) {
    const floatx4 x = *reinterpret_cast<const floatx4*>(dzp + c), y = *reinterpret_cast<const floatx4*>(zp + c);
    s = __builtin_fmaf(x[0], y[0], s);
    s = __builtin_fmaf(x[1], y[1], s);
    s = __builtin_fmaf(x[2], y[2], s);
    s = __builtin_fmaf(x[3], y[3], s);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) delta[((int64_t)b * 16 + h) * Lq + i] = s;
}

// out[n] = sum_s part[s][n] in split order, 4 floats per thread (count a multiple of 4, 16-byte aligned buffers)
__global__ __launch_bounds__(256) void khf_split_sum_kernel(const float* part, int64_t split_stride, int splits,
                                                            int64_t count, float* out) {
  const int64_t n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (n >= count) return;
  floatx4 s = *reinterpret_cast<const floatx4*>(part + n);
  for (int p = 1; p < splits; ++p) s += *reinterpret_cast<const floatx4*>(part + (int64_t)p * split_stride + n);
  *reinterpret_cast<floatx4*>(out + n) = s;
}

inline bool kf_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int kf_check(const void* q, int64_t q_sb, int64_t q_si, int64_t q_sh, const void* k, int64_t k_sb, int64_t k_sn,
             const void* v, int64_t v_sb, int64_t v_sn, int B, int Lq, int N, int R, int heads) {
  HLA_REQUIRE(B >= 1 && B <= 65535 && Lq >= 0 && N >= 1, HLA_S6_EINVAL, "khop_f32: bad sizes B=%d Lq=%d N=%d", B,
              Lq, N);
  HLA_REQUIRE(heads == 16, HLA_S6_EUNSUPPORTED, "khop_f32: %d query heads (16 supported)", heads);
  HLA_REQUIRE(R == 128 || R == 256 || R == 512 || R == 1024, HLA_S6_EUNSUPPORTED,
              "khop_f32: latent width %d not in {128, 256, 512, 1024}", R);
  HLA_REQUIRE(q && k && v, HLA_S6_EINVAL, "khop_f32: null input");
  HLA_REQUIRE(kf_aligned16(q) && kf_aligned16(k) && kf_aligned16(v) && q_sb % 4 == 0 && q_si % 4 == 0 &&
                  q_sh % 4 == 0 && k_sb % 4 == 0 && k_sn % 4 == 0 && v_sb % 4 == 0 && v_sn % 4 == 0,
              HLA_S6_EINVAL, "khop_f32: q/k/v rows must be 16-byte aligned with a unit last stride");
  return HLA_S6_OK;
}

// Columns per wave of each kernel and width (forward: 256 from width 256 up; dq and dk / dv: 128).
#define HLA_KF_LAUNCH(KERNEL, R, RC, W, GRID, P, ST) \
  hipLaunchKernelGGL((KERNEL<R, RC, W>), GRID, dim3(64 * (W)), 0, ST, P)

int kf_groups(int R, int RC, int W) { return W / (R / RC); }
int kf_fwd_rc(int R) { return R >= 256 ? 256 : 128; }
// dq and dk / dv: 8 waves of 128 columns. (At width 1024 these spill: the next step's 128 KB tile in flight beside
// the resident operands and accumulators exceeds two waves' registers per SIMD; 16 waves of 64 columns spill more.)
int kf_bwd_rc(int) { return 128; }
int kf_bwd_waves(int) { return 8; }

}  // namespace
}  // namespace hla

extern "C" int hla_s6_khop_forward_f32(const float* q, int64_t q_sb, int64_t q_si, int64_t q_sh, const float* k,
                                       int64_t k_sb, int64_t k_sn, const float* v, int64_t v_sb, int64_t v_sn,
                                       const uint8_t* mask, int64_t m_sb, int64_t m_si, const int32_t* bound,
                                       int32_t B, int32_t Lq, int32_t N, int32_t heads, int32_t width, float scale,
                                       float* z, int64_t z_sb, int64_t z_si, int64_t z_sh, float* lse, void* stream) {
  using namespace hla;
  int rc = kf_check(q, q_sb, q_si, q_sh, k, k_sb, k_sn, v, v_sb, v_sn, B, Lq, N, width, heads);
  if (rc != HLA_S6_OK) return rc;
  if (Lq == 0) return HLA_S6_OK;
  HLA_REQUIRE(bound && z && lse, HLA_S6_EINVAL, "khop_forward_f32: null bound / output");
  HLA_REQUIRE(kf_aligned16(z) && z_sb % 4 == 0 && z_si % 4 == 0 && z_sh % 4 == 0, HLA_S6_EINVAL,
              "khop_forward_f32: z rows must be 16-byte aligned with a unit last stride");
  KfParams p = {};
  p.q = q; p.q_sb = q_sb; p.q_si = q_si; p.q_sh = q_sh;
  p.k = k; p.v = v; p.k_sb = k_sb; p.k_sn = k_sn; p.v_sb = v_sb; p.v_sn = v_sn;
  p.mask = mask; p.m_sb = m_sb; p.m_si = m_si;
  p.bound = bound;
  p.B = B; p.Lq = Lq; p.N = N;
  p.scale = scale;
  p.scale_log2 = scale * kLog2e;
  p.z = z; p.z_sb = z_sb; p.z_si = z_si; p.z_sh = z_sh;
  p.lse = lse;
  hipStream_t st = as_stream(stream);
  const int rcw = kf_fwd_rc(width), tg = kf_groups(width, rcw, 8);
  const dim3 grid((unsigned)((Lq + tg - 1) / tg), (unsigned)B);
  switch (width) {
    case 128: HLA_KF_LAUNCH(khf_fwd, 128, 128, 8, grid, p, st); break;
    case 256: HLA_KF_LAUNCH(khf_fwd, 256, 256, 8, grid, p, st); break;
    case 512: HLA_KF_LAUNCH(khf_fwd, 512, 256, 8, grid, p, st); break;
    default: HLA_KF_LAUNCH(khf_fwd, 1024, 256, 8, grid, p, st); break;
  }
  return check_launch("khop_forward_f32");
}

extern "C" int64_t hla_s6_khop_backward_f32_workspace(int32_t B, int32_t Lq, int32_t N, int32_t width,
                                                       int32_t key_splits) {
  if (B < 1 || Lq < 0 || N < 1 || width < 1 || key_splits < 1) return 0;
  return key_splits > 1 ? 2 * (int64_t)key_splits * B * N * width : 0;
}

extern "C" int hla_s6_khop_backward_f32(const float* q, int64_t q_sb, int64_t q_si, int64_t q_sh, const float* k,
                                        int64_t k_sb, int64_t k_sn, const float* v, int64_t v_sb, int64_t v_sn,
                                        const uint8_t* mask, int64_t m_sb, int64_t m_si, const int32_t* bound,
                                        int32_t B, int32_t Lq, int32_t N, int32_t heads, int32_t width, float scale,
                                        const float* z, int64_t z_sb, int64_t z_si, int64_t z_sh, const float* lse,
                                        const float* dz, int64_t dz_sb, int64_t dz_si, int64_t dz_sh,
                                        const float* dlse, float* delta, float* dq, int64_t dq_sb, int64_t dq_si,
                                        int64_t dq_sh, float* dk, int64_t dk_sb, int64_t dk_sn, float* dv,
                                        int64_t dv_sb, int64_t dv_sn, int32_t key_splits, float* workspace,
                                        int64_t workspace_floats, void* stream) {
  using namespace hla;
  int rc = kf_check(q, q_sb, q_si, q_sh, k, k_sb, k_sn, v, v_sb, v_sn, B, Lq, N, width, heads);
  if (rc != HLA_S6_OK) return rc;
  HLA_REQUIRE(bound && z && lse && dz && delta, HLA_S6_EINVAL, "khop_backward_f32: null input");
  HLA_REQUIRE(key_splits >= 1 && key_splits <= 64, HLA_S6_EINVAL,
              "khop_backward_f32: key_splits %d not in [1, 64]", key_splits);
  HLA_REQUIRE(kf_aligned16(dz) && dz_sb % 4 == 0 && dz_si % 4 == 0 && dz_sh % 4 == 0 && kf_aligned16(z) &&
                  z_sb % 4 == 0 && z_si % 4 == 0 && z_sh % 4 == 0,
              HLA_S6_EINVAL, "khop_backward_f32: z / dz rows must be 16-byte aligned with a unit last stride");
  const bool need_q = dq != nullptr, need_kv = dk != nullptr || dv != nullptr;
  HLA_REQUIRE(!need_kv || (dk && dv), HLA_S6_EINVAL, "khop_backward_f32: dk and dv come together");
  HLA_REQUIRE(!need_q || (kf_aligned16(dq) && dq_sb % 4 == 0 && dq_si % 4 == 0 && dq_sh % 4 == 0), HLA_S6_EINVAL,
              "khop_backward_f32: dq rows must be 16-byte aligned with a unit last stride");
  const int64_t part = (int64_t)B * N * width;
  const bool split = need_kv && key_splits > 1;
  if (split) {
    HLA_REQUIRE(workspace && kf_aligned16(workspace) && workspace_floats >= 2 * key_splits * part, HLA_S6_EWORKSPACE,
                "khop_backward_f32: %d key splits need a workspace of %lld floats (got %lld)", key_splits,
                (long long)(2 * key_splits * part), (long long)workspace_floats);
    HLA_REQUIRE(dk_sb == (int64_t)N * width && dk_sn == width && dv_sb == (int64_t)N * width && dv_sn == width &&
                    kf_aligned16(dk) && kf_aligned16(dv),
                HLA_S6_EINVAL, "khop_backward_f32: with key splits dk / dv must be contiguous [B, N, width]");
  }
  HLA_REQUIRE(!need_kv || split || (kf_aligned16(dk) && kf_aligned16(dv) && dk_sb % 4 == 0 && dk_sn % 4 == 0 &&
                                    dv_sb % 4 == 0 && dv_sn % 4 == 0),
              HLA_S6_EINVAL, "khop_backward_f32: dk / dv rows must be 16-byte aligned with a unit last stride");
  hipStream_t st = as_stream(stream);
  KfParams p = {};
  p.q = q; p.q_sb = q_sb; p.q_si = q_si; p.q_sh = q_sh;
  p.k = k; p.v = v; p.k_sb = k_sb; p.k_sn = k_sn; p.v_sb = v_sb; p.v_sn = v_sn;
  p.mask = mask; p.m_sb = m_sb; p.m_si = m_si;
  p.bound = bound;
  p.B = B; p.Lq = Lq; p.N = N;
  p.scale = scale;
  p.scale_log2 = scale * kLog2e;
  p.lse = const_cast<float*>(lse);
  p.dz = dz; p.dz_sb = dz_sb; p.dz_si = dz_si; p.dz_sh = dz_sh;
  p.dlse = dlse;
  p.delta = delta;
  if (Lq > 0) {
    const int64_t rows = (int64_t)B * Lq * 16;
    hipLaunchKernelGGL(khf_delta_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, dz, dz_sb, dz_si, dz_sh,
                       z, z_sb, z_si, z_sh, B, Lq, width, delta);
    if ((rc = check_launch("khop_delta_f32")) != HLA_S6_OK) return rc;
  }
  if (need_q && Lq > 0) {
    p.dq = dq; p.dq_sb = dq_sb; p.dq_si = dq_si; p.dq_sh = dq_sh;
    const int tg = kf_groups(width, kf_bwd_rc(width), kf_bwd_waves(width));
    const dim3 grid((unsigned)((Lq + tg - 1) / tg), (unsigned)B);
    switch (width) {
      case 128: HLA_KF_LAUNCH(khf_dq, 128, 128, 8, grid, p, st); break;
      case 256: HLA_KF_LAUNCH(khf_dq, 256, 128, 8, grid, p, st); break;
      case 512: HLA_KF_LAUNCH(khf_dq, 512, 128, 8, grid, p, st); break;
      default: HLA_KF_LAUNCH(khf_dq, 1024, 128, 8, grid, p, st); break;
    }
    if ((rc = check_launch("khop_dq_f32")) != HLA_S6_OK) return rc;
  }
  if (need_kv) {
    p.key_splits = key_splits;
    p.kv_ss = part;
    p.dk = split ? workspace : dk;
    p.dv = split ? workspace + key_splits * part : dv;
    p.dk_sb = split ? (int64_t)N * width : dk_sb;
    p.dk_sn = split ? width : dk_sn;
    p.dv_sb = split ? (int64_t)N * width : dv_sb;
    p.dv_sn = split ? width : dv_sn;
    const int keys = 16 * kf_groups(width, kf_bwd_rc(width), kf_bwd_waves(width));
    const dim3 grid((unsigned)((N + keys - 1) / keys), (unsigned)B, (unsigned)key_splits);
    switch (width) {
      case 128: HLA_KF_LAUNCH(khf_dkdv, 128, 128, 8, grid, p, st); break;
      case 256: HLA_KF_LAUNCH(khf_dkdv, 256, 128, 8, grid, p, st); break;
      case 512: HLA_KF_LAUNCH(khf_dkdv, 512, 128, 8, grid, p, st); break;
      default: HLA_KF_LAUNCH(khf_dkdv, 1024, 128, 8, grid, p, st); break;
    }
    if ((rc = check_launch("khop_dkdv_f32")) != HLA_S6_OK) return rc;
    if (split) {
      const unsigned blocks = (unsigned)((part / 4 + 255) / 256);
      hipLaunchKernelGGL(khf_split_sum_kernel, dim3(blocks), dim3(256), 0, st, workspace, part, key_splits, part, dk);
      hipLaunchKernelGGL(khf_split_sum_kernel, dim3(blocks), dim3(256), 0, st, workspace + key_splits * part, part,
                         key_splits, part, dv);
      if ((rc = check_launch("khop_split_sum_f32")) != HLA_S6_OK) return rc;
    }
  }
  return HLA_S6_OK;
}
