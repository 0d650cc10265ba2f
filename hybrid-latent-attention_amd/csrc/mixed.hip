// The LSE merge and B_t projection of the HF rolling engine's joint attention (hla/latent/batched_engine.py:154-182).
//
// The engine's one softmax over [latent history rows of K blocks || the exact current chunk] is computed as parts:
// the chunk gives (o_c [B,H,n,128] fp32, lse_c), block p gives (z_p [B,H,n,R] bf16, lse_p) normalized in latent
// space. With w_j = exp(lse_j - logsumexp(lse_c, lse_0, ..)) the joint output is
//   out = w_c o_c + bf16(sum_p w_p z_p) @ B_t[h]                                   (bf16 result, fp32 sums)
// (the reference rounds the joint latent output z to bf16 before its product with B_t, batched_engine.py:177-180).
// The finite values these kernels round to bf16 (z, out, d z) take the hardware conversion (round to nearest even).
//
// merge_fwd: one workgroup per (64 queries, head, 64 output columns), the two column blocks of a query block on one
// XCD (8 workgroups apart in dispatch order); 4 waves of 16 queries x 4 column tiles on
// v_mfma_f32_16x16x32_bf16. Every global load is issued before the first barrier: the B_t slab B[h, :, 64 columns]
// (into LDS row-major, rows 72 elements apart; the B operand comes back by two ds_read_b64_tr_b16 per step), the
// lse of the wave's queries and the parts' z rows (the A operand: the lane's query, 8 consecutive latent columns per
// k-step, weighted and summed in fp32, rounded once to bf16), and the chunk output of the lane's output rows.
//
// merge_bwd: for the cotangent dout [B,H,n,128] (bf16) of out, with g = dout @ B_t[h]^T [R] per query,
//   d o_c = w_c dout,  d z_p = w_p g,  d lse_j = w_j (a_j - D)
// where a_c = <dout, o_c>, a_p = <g, z_p> and D = w_c a_c + sum_p w_p a_p (= <dout, out>). One wave per 16 queries of
// one head, all R columns: g^T = B[h] . dout^T on 16x16x32 MFMA, whose A operand (16 latent rows x 8 consecutive
// head-dim columns per lane) is a contiguous 16-byte piece of B[h]'s rows and whose B operand is the lane's query's
// dout row piece, so each lane ends up holding 4 consecutive latent columns of g for its own query: d z_p and the
// z_p reads of a_p are 8-byte accesses, and the per-query sums are reductions over the lane's 4 lane groups.
#include "common.h"

namespace hla {
namespace {

constexpr int kMixD = 128;      // head dim of o_c, dout and out
constexpr int kMixParts = 8;    // history blocks per call

struct MixedParams {
  int B, H, n, parts;
  const float* oc;  // [B,H,n,128] fp32
  int64_t oc_sb, oc_sh, oc_si;
  const float* lc;  // [B,H,n] fp32 contiguous
  const uint16_t* z[kMixParts];  // [B,H,n,R] bf16, unit last stride
  int64_t z_sb[kMixParts], z_sh[kMixParts], z_si[kMixParts];
  const float* lz[kMixParts];  // [B,H,n] fp32 contiguous
  const uint16_t* Bw;  // [H,R,128] bf16
  int64_t b_sh, b_sr;
  // forward
  uint16_t* out;  // [B,H,n,128] bf16
  int64_t o_sb, o_sh, o_si;
  // backward
  const uint16_t* dout;  // [B,H,n,128] bf16
  int64_t do_sb, do_sh, do_si;
  float* doc;  // [B,H,n,128] fp32
  int64_t doc_sb, doc_sh, doc_si;
  float* dlc;  // [B,H,n] fp32 contiguous
  uint16_t* dz[kMixParts];  // like z
  int64_t dz_sb[kMixParts], dz_sh[kMixParts], dz_si[kMixParts];
  float* dlz[kMixParts];  // [B,H,n] fp32 contiguous
};

// lse of query q (= b * n + i) of head h: l[0] of the chunk, l[1 + p] of block p (-inf past the blocks). Every
// load is unconditional (the host points the unused block slots at valid memory) so that they all issue before the
// first wait.
__device__ __forceinline__ void mixed_lse(const MixedParams& a, int q, int h, float (&l)[1 + kMixParts]) {
  const int64_t row = (int64_t)(q / a.n) * a.H * a.n + (int64_t)h * a.n + q % a.n;
  l[0] = a.lc[row];
  float v[kMixParts];
#pragma unroll
  for (int p = 0; p < kMixParts; ++p) v[p] = a.lz[p][row];
#pragma unroll
  for (int p = 0; p < kMixParts; ++p) l[1 + p] = p < a.parts ? v[p] : -INFINITY;
}

// Joint-softmax weights from those lse: w_j = exp(l_j - logsumexp(l)). A block whose query sees no row
// (lse = -inf) weighs 0; a query with no key at all gets all-zero weights.
__device__ __forceinline__ void mixed_weights(const float (&l)[1 + kMixParts], float (&w)[1 + kMixParts]) {
  float m = l[0];
#pragma unroll
  for (int j = 1; j <= kMixParts; ++j) m = fmaxf(m, l[j]);
  if (m == -INFINITY) {
#pragma unroll
    for (int j = 0; j <= kMixParts; ++j) w[j] = 0.f;
    return;
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j <= kMixParts; ++j) s += l[j] == -INFINITY ? 0.f : expf(l[j] - m);
  const float total = m + logf(s);
#pragma unroll
  for (int j = 0; j <= kMixParts; ++j) w[j] = l[j] == -INFINITY ? 0.f : expf(l[j] - total);
}

// The lane's 8 bf16 z values (one 16-byte piece) of blocks 0 and 1, weighted, plus those of blocks 2.. loaded here.
__device__ __forceinline__ u32x4 mixed_piece(const MixedParams& a, u32x4 z0, u32x4 z1, const float (&w)[1 + kMixParts],
                                             int64_t b, int h, int64_t i, int col, bool live) {
  float f[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __builtin_fmaf(w[2], lo_bf(z1[e]), w[1] * lo_bf(z0[e]));
    f[2 * e + 1] = __builtin_fmaf(w[2], hi_bf(z1[e]), w[1] * hi_bf(z0[e]));
  }
  for (int p = 2; p < a.parts; ++p) {
    const u32x4 zp = live ? ld16(a.z[p] + b * a.z_sb[p] + (int64_t)h * a.z_sh[p] + i * a.z_si[p] + col)
                          : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = __builtin_fmaf(w[1 + p], lo_bf(zp[e]), f[2 * e]);
      f[2 * e + 1] = __builtin_fmaf(w[1 + p], hi_bf(zp[e]), f[2 * e + 1]);
    }
  }
  return u32x4{pack2_hw(f[0], f[1]), pack2_hw(f[2], f[3]), pack2_hw(f[4], f[5]), pack2_hw(f[6], f[7])};
}

template <int R>
__global__ __launch_bounds__(256) void merge_fwd(MixedParams a) {
  constexpr int LS = 72;      // LDS row stride of the slab (one latent row per LDS row, 64 columns + 8), bf16
  constexpr int CH = R / 32;  // 16-byte slab pieces per thread (R rows x 8 pieces / 256 threads) = MFMA k-steps
  extern __shared__ __attribute__((aligned(16))) uint16_t wt[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, g = lane >> 4;
  // workgroup L takes column block (L / 8) % 2 of the (head, query block) pair (L % 8) + 8 (L / 16): the two column
  // blocks of a query block are 8 workgroups apart, so they run on one XCD and the second reads z from its L2
  const int L = blockIdx.x;
  const int pair = (L & 7) + 8 * (L >> 4);
  const int h = pair % a.H, c0 = ((L >> 3) & 1) * 64;
  const int Q = a.B * a.n;
  const int q0 = (pair / a.H) * 64 + wave * 16;
  if (q0 - wave * 16 >= Q) return;  // past the last query block (uniform over the workgroup)

  // every global load before the first use: the slab, the lse of the A row and of the 4 output rows, blocks 0 and
  // 1 of the A row (query qa, latent columns 32 kk + 8 g .. + 8), o_c of the output rows
  const uint16_t* bh = a.Bw + (int64_t)h * a.b_sh + c0;
  u32x4 slab[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = i * 256 + tid;
    slab[i] = ld16(bh + (int64_t)(c >> 3) * a.b_sr + (c & 7) * 8);
  }
  const int qa = q0 + l16;
  const bool a_live = qa < Q;
  const int64_t ab = (a_live ? qa : 0) / a.n, ai = (a_live ? qa : 0) % a.n;
  float la[1 + kMixParts];
  mixed_lse(a, a_live ? qa : Q - 1, h, la);
  float lr[4][1 + kMixParts];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int q = q0 + 4 * g + r;
    mixed_lse(a, q < Q ? q : Q - 1, h, lr[r]);
  }
  // (block 1's slot holds block 0 when there is one block: its weight is then 0; dead lanes read query 0)
  const uint16_t* zr0 = a.z[0] + ab * a.z_sb[0] + (int64_t)h * a.z_sh[0] + ai * a.z_si[0] + 8 * g;
  const uint16_t* zr1 = a.z[1] + ab * a.z_sb[1] + (int64_t)h * a.z_sh[1] + ai * a.z_si[1] + 8 * g;
  u32x4 z0[CH], z1[CH];
#pragma unroll
  for (int kk = 0; kk < CH; ++kk) {
    z0[kk] = ld16(zr0 + 32 * kk);
    z1[kk] = ld16(zr1 + 32 * kk);
  }
  float ocv[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int q = q0 + 4 * g + r;
    const bool live = q < Q;
    const int64_t b = (live ? q : 0) / a.n, i = (live ? q : 0) % a.n;
    const float* orow = a.oc + b * a.oc_sb + (int64_t)h * a.oc_sh + i * a.oc_si + c0 + l16;
#pragma unroll
    for (int t = 0; t < 4; ++t) ocv[r][t] = orow[16 * t];
  }
  // the slab into LDS: wt[k][local column]
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = i * 256 + tid;
    st16(wt + (c >> 3) * LS + (c & 7) * 8, slab[i]);
  }
  float wa[1 + kMixParts];
  mixed_weights(la, wa);
  if (!a_live) {
#pragma unroll
    for (int j = 0; j <= kMixParts; ++j) wa[j] = 0.f;
  }
  u32x4 xa[CH];
#pragma unroll
  for (int kk = 0; kk < CH; ++kk) xa[kk] = mixed_piece(a, z0[kk], z1[kk], wa, ab, h, ai, 32 * kk + 8 * g, a_live);
  float wc[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float w[1 + kMixParts];
    mixed_weights(lr[r], w);
    wc[r] = w[0];
  }
  __syncthreads();

  floatx4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  // B operand of lane (g, l16): wt[32 kk + 8 g + e][16 t + l16], e < 8 (the transposing read hands lane l16 its
  // column of the 4 rows its 16-lane group addresses)
  const uint16_t* tp = wt + (8 * g + (l16 >> 2)) * LS + 4 * (l16 & 3);
#pragma unroll
  for (int kk = 0; kk < CH; ++kk) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint16_t* p = tp + 32 * kk * LS + 16 * t;
      const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)p);
      const short4v hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)(p + 4 * LS));
      acc[t] = mfma16x16x32(xa[kk], join_tr(lo, hi), acc[t]);
    }
  }

  // lane holds (z @ B)[q0 + 4 g + r][c0 + 16 t + l16]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int q = q0 + 4 * g + r;
    if (q >= Q) continue;
    const int64_t b = q / a.n, i = q % a.n;
    uint16_t* orow = a.out + b * a.o_sb + (int64_t)h * a.o_sh + i * a.o_si + c0 + l16;
#pragma unroll
    for (int t = 0; t < 4; ++t) orow[16 * t] = (uint16_t)pack2_hw(__builtin_fmaf(wc[r], ocv[r][t], acc[t][r]), 0.f);
  }
}

// Backward in phases, each issuing all of its loads before its first wait (stores to d z would otherwise keep
// the compiler from moving later loads above them: one memory latency per tile):
//   1. dout and o_c of the lane's query, the lse of its parts; a_c;
//   2. g^T = B[h] . dout^T for every 16-row latent tile (loads of B only);
//   3. per block: its z over the lane's columns, then a_p and the d z stores;
//   4. d o_c and the d lse.
template <int R>
__global__ __launch_bounds__(256) void merge_bwd(MixedParams a) {
  constexpr int NT = R / 16;  // 16-row latent tiles of g
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, g = lane >> 4;
  const int h = blockIdx.y;
  const int Q = a.B * a.n;
  const int q = blockIdx.x * 64 + wave * 16 + l16;  // the lane's query
  const bool live = q < Q;
  const int64_t b = (live ? q : 0) / a.n, i = (live ? q : 0) % a.n;  // dead lanes read query 0 and store nothing

  // 1. dout row piece of the lane's query: head-dim columns 32 kk + 8 g .. + 8 (the MFMA B operand), o_c there
  const uint16_t* dr = a.dout + b * a.do_sb + (int64_t)h * a.do_sh + i * a.do_si + 8 * g;
  const float* orow = a.oc + b * a.oc_sb + (int64_t)h * a.oc_sh + i * a.oc_si + 8 * g;
  u32x4 dv[4];
  floatx4 ov[4][2];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    dv[kk] = ld16(dr + 32 * kk);
    ov[kk][0] = *reinterpret_cast<const floatx4*>(orow + 32 * kk);
    ov[kk][1] = *reinterpret_cast<const floatx4*>(orow + 32 * kk + 4);
  }
  float l[1 + kMixParts], w[1 + kMixParts];
  mixed_lse(a, live ? q : Q - 1, h, l);
  mixed_weights(l, w);
  floatx4 dd[4][2];  // dout in fp32
  float ac = 0.f;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      dd[kk][0][2 * e] = lo_bf(dv[kk][e]);
      dd[kk][0][2 * e + 1] = hi_bf(dv[kk][e]);
      dd[kk][1][2 * e] = lo_bf(dv[kk][2 + e]);
      dd[kk][1][2 * e + 1] = hi_bf(dv[kk][2 + e]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      ac = __builtin_fmaf(dd[kk][0][e], ov[kk][0][e], __builtin_fmaf(dd[kk][1][e], ov[kk][1][e], ac));
  }
  ac = wave_sum16x4(ac);

  // 2. g^T tiles: lane (g, l16) holds g[q][16 t + 4 g + rr]
  const uint16_t* bh = a.Bw + (int64_t)h * a.b_sh + (int64_t)l16 * a.b_sr + 8 * g;
  floatx4 gacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint16_t* br = bh + (int64_t)(16 * t) * a.b_sr;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) acc = mfma16x16x32(ld16(br + 32 * kk), dv[kk], acc);
    gacc[t] = acc;
  }

  // 3. per block: a_p = <g, z_p> and d z_p = bf16(w_p g)
  float ap[kMixParts];
#pragma unroll
  for (int p = 0; p < kMixParts; ++p) ap[p] = 0.f;
#pragma unroll
  for (int p = 0; p < kMixParts; ++p) {
    if (p >= a.parts) break;
    const uint16_t* zr = a.z[p] + b * a.z_sb[p] + (int64_t)h * a.z_sh[p] + i * a.z_si[p] + 4 * g;
    uint2 zz[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) zz[t] = *reinterpret_cast<const uint2*>(zr + 16 * t);
    float sdot = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const floatx4 gt = gacc[t];
      sdot = __builtin_fmaf(gt[0], lo_bf(zz[t].x), sdot);
      sdot = __builtin_fmaf(gt[1], hi_bf(zz[t].x), sdot);
      sdot = __builtin_fmaf(gt[2], lo_bf(zz[t].y), sdot);
      sdot = __builtin_fmaf(gt[3], hi_bf(zz[t].y), sdot);
    }
    ap[p] = wave_sum16x4(sdot);
    if (live) {
      const float wp = w[1 + p];
      uint16_t* dzr = a.dz[p] + b * a.dz_sb[p] + (int64_t)h * a.dz_sh[p] + i * a.dz_si[p] + 4 * g;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const floatx4 gt = gacc[t];
        *reinterpret_cast<uint2*>(dzr + 16 * t) =
            uint2{pack2_hw(gt[0] * wp, gt[1] * wp), pack2_hw(gt[2] * wp, gt[3] * wp)};
      }
    }
  }

  // 4. d o_c = w_c dout, d lse_j = w_j (a_j - D)
  if (!live) return;
  float* drow = a.doc + b * a.doc_sb + (int64_t)h * a.doc_sh + i * a.doc_si + 8 * g;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    *reinterpret_cast<floatx4*>(drow + 32 * kk) = dd[kk][0] * w[0];
    *reinterpret_cast<floatx4*>(drow + 32 * kk + 4) = dd[kk][1] * w[0];
  }
  if (g != 0) return;
  float D = w[0] * ac;
#pragma unroll
  for (int p = 0; p < kMixParts; ++p)
    if (p < a.parts) D = __builtin_fmaf(w[1 + p], ap[p], D);
  const int64_t row = b * a.H * a.n + (int64_t)h * a.n + i;
  a.dlc[row] = w[0] * (ac - D);
#pragma unroll
  for (int p = 0; p < kMixParts; ++p)
    if (p < a.parts) a.dlz[p][row] = w[1 + p] * (ap[p] - D);
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int fill_mixed(MixedParams& m, int32_t batch, int32_t heads, int32_t chunk, int32_t width, int32_t head_dim,
               const float* oc, int64_t oc_sb, int64_t oc_sh, int64_t oc_si, const float* lse_c, int32_t parts,
               const void* const* z, const int64_t* z_strides, const float* const* lse_z, const void* Bt,
               int64_t b_sh, int64_t b_sr) {
  HLA_REQUIRE(batch >= 0 && chunk >= 0 && heads >= 1 && heads <= 65535, HLA_S6_EINVAL,
              "mixed_merge: bad batch, chunk or head count");
  HLA_REQUIRE(width == 256 || width == 512, HLA_S6_EUNSUPPORTED, "mixed_merge: latent width %d not in {256, 512}",
              width);
  HLA_REQUIRE(head_dim == kMixD, HLA_S6_EUNSUPPORTED, "mixed_merge: head_dim %d (the kernels are built for 128)",
              head_dim);
  HLA_REQUIRE(parts >= 1 && parts <= kMixParts, HLA_S6_EUNSUPPORTED,
              "mixed_merge: %d history blocks (1 to %d per call)", parts, kMixParts);
  const int64_t Q = (int64_t)batch * chunk;
  HLA_REQUIRE((Q + 63) / 64 <= 65535 && (int64_t)heads * ((Q + 63) / 64) <= (1ll << 30), HLA_S6_EUNSUPPORTED,
              "mixed_merge: %lld queries x %d heads exceed the grid", (long long)Q, heads);
  m = MixedParams{};
  m.B = batch;
  m.H = heads;
  m.n = chunk;
  m.parts = parts;
  if (Q == 0) return HLA_S6_OK;
  HLA_REQUIRE(oc && lse_c && Bt && z && z_strides && lse_z, HLA_S6_EINVAL,
              "mixed_merge: null pointer argument");
  HLA_REQUIRE(al16(oc) && oc_sb % 4 == 0 && oc_sh % 4 == 0 && oc_si % 4 == 0, HLA_S6_EINVAL,
              "mixed_merge: o_c rows must be 16-byte aligned with a unit last stride");
  HLA_REQUIRE(al16(Bt) && b_sh % 8 == 0 && b_sr % 8 == 0, HLA_S6_EINVAL,
              "mixed_merge: B_t rows must be 16-byte aligned with a unit last stride");
  m.oc = oc;
  m.oc_sb = oc_sb;
  m.oc_sh = oc_sh;
  m.oc_si = oc_si;
  m.lc = lse_c;
  for (int p = 0; p < parts; ++p) {
    HLA_REQUIRE(z[p] && lse_z[p], HLA_S6_EINVAL, "mixed_merge: null pointer for block %d", p);
    const int64_t sb = z_strides[3 * p], sh = z_strides[3 * p + 1], si = z_strides[3 * p + 2];
    HLA_REQUIRE(al16(z[p]) && sb % 8 == 0 && sh % 8 == 0 && si % 8 == 0, HLA_S6_EINVAL,
                "mixed_merge: z rows of block %d must be 16-byte aligned with a unit last stride", p);
    m.z[p] = static_cast<const uint16_t*>(z[p]);
    m.z_sb[p] = sb;
    m.z_sh[p] = sh;
    m.z_si[p] = si;
    m.lz[p] = lse_z[p];
  }
  for (int p = parts; p < kMixParts; ++p) {  // unused slots: valid memory for the kernels' unconditional loads
    m.z[p] = parts > 0 ? m.z[0] : nullptr;
    m.z_sb[p] = m.z_sb[0];
    m.z_sh[p] = m.z_sh[0];
    m.z_si[p] = m.z_si[0];
    m.lz[p] = lse_c;
  }
  m.Bw = static_cast<const uint16_t*>(Bt);
  m.b_sh = b_sh;
  m.b_sr = b_sr;
  return HLA_S6_OK;
}

}  // namespace
}  // namespace hla

extern "C" int hla_s6_mixed_merge_forward(int32_t batch, int32_t num_heads, int32_t chunk, int32_t width,
                                          int32_t head_dim, const float* o_c, int64_t oc_sb, int64_t oc_sh,
                                          int64_t oc_si, const float* lse_c, int32_t parts, const void* const* z,
                                          const int64_t* z_strides, const float* const* lse_z, const void* Bt,
                                          int64_t b_sh, int64_t b_sr, void* out, int64_t o_sb, int64_t o_sh,
                                          int64_t o_si, void* stream) {
  using namespace hla;
  MixedParams m;
  int rc = fill_mixed(m, batch, num_heads, chunk, width, head_dim, o_c, oc_sb, oc_sh, oc_si, lse_c, parts, z,
                      z_strides, lse_z, Bt, b_sh, b_sr);
  if (rc != HLA_S6_OK || (int64_t)batch * chunk == 0) return rc;
  HLA_REQUIRE(out, HLA_S6_EINVAL, "mixed_merge_forward: null output");
  m.out = static_cast<uint16_t*>(out);
  m.o_sb = o_sb;
  m.o_sh = o_sh;
  m.o_si = o_si;
  // 2 column blocks x heads x query blocks, numbered as the kernel decodes them (rounded up to whole groups of 16)
  const int64_t pairs = (int64_t)num_heads * (((int64_t)batch * chunk + 63) / 64);
  const dim3 grid((unsigned)((pairs + 7) / 8 * 16));
  const hipStream_t st = as_stream(stream);
  if (width == 512) {
    constexpr int lds = 512 * 72 * 2;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&merge_fwd<512>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return fail(HLA_S6_ELAUNCH, "mixed_merge_forward: LDS size %d rejected", lds);
    hipLaunchKernelGGL(merge_fwd<512>, grid, dim3(256), lds, st, m);
  } else {
    hipLaunchKernelGGL(merge_fwd<256>, grid, dim3(256), 256 * 72 * 2, st, m);
  }
  return check_launch("mixed_merge_forward");
}

extern "C" int hla_s6_mixed_merge_backward(
    int32_t batch, int32_t num_heads, int32_t chunk, int32_t width, int32_t head_dim, const float* o_c, int64_t oc_sb,
    int64_t oc_sh, int64_t oc_si, const float* lse_c, int32_t parts, const void* const* z, const int64_t* z_strides,
    const float* const* lse_z, const void* Bt, int64_t b_sh, int64_t b_sr, const void* dout, int64_t do_sb,
    int64_t do_sh, int64_t do_si, float* d_oc, int64_t doc_sb, int64_t doc_sh, int64_t doc_si, float* d_lse_c,
    void* const* dz, const int64_t* dz_strides, float* const* d_lse_z, void* stream) {
  using namespace hla;
  MixedParams m;
  int rc = fill_mixed(m, batch, num_heads, chunk, width, head_dim, o_c, oc_sb, oc_sh, oc_si, lse_c, parts, z,
                      z_strides, lse_z, Bt, b_sh, b_sr);
  if (rc != HLA_S6_OK || (int64_t)batch * chunk == 0) return rc;
  HLA_REQUIRE(dout && d_oc && d_lse_c && dz && dz_strides && d_lse_z, HLA_S6_EINVAL,
              "mixed_merge_backward: null pointer argument");
  HLA_REQUIRE(al16(dout) && do_sb % 8 == 0 && do_sh % 8 == 0 && do_si % 8 == 0, HLA_S6_EINVAL,
              "mixed_merge_backward: dout rows must be 16-byte aligned with a unit last stride");
  HLA_REQUIRE(al16(d_oc) && doc_sb % 4 == 0 && doc_sh % 4 == 0 && doc_si % 4 == 0, HLA_S6_EINVAL,
              "mixed_merge_backward: d o_c rows must be 16-byte aligned with a unit last stride");
  m.dout = static_cast<const uint16_t*>(dout);
  m.do_sb = do_sb;
  m.do_sh = do_sh;
  m.do_si = do_si;
  m.doc = d_oc;
  m.doc_sb = doc_sb;
  m.doc_sh = doc_sh;
  m.doc_si = doc_si;
  m.dlc = d_lse_c;
  for (int p = 0; p < parts; ++p) {
    HLA_REQUIRE(dz[p] && d_lse_z[p], HLA_S6_EINVAL, "mixed_merge_backward: null gradient pointer for block %d", p);
    const int64_t sb = dz_strides[3 * p], sh = dz_strides[3 * p + 1], si = dz_strides[3 * p + 2];
    HLA_REQUIRE((reinterpret_cast<uintptr_t>(dz[p]) & 7u) == 0 && sb % 4 == 0 && sh % 4 == 0 && si % 4 == 0,
                HLA_S6_EINVAL, "mixed_merge_backward: dz rows of block %d must be 8-byte aligned", p);
    m.dz[p] = static_cast<uint16_t*>(dz[p]);
    m.dz_sb[p] = sb;
    m.dz_sh[p] = sh;
    m.dz_si[p] = si;
    m.dlz[p] = d_lse_z[p];
  }
  const dim3 grid((unsigned)(((int64_t)batch * chunk + 63) / 64), (unsigned)num_heads);
  const hipStream_t st = as_stream(stream);
  if (width == 512) hipLaunchKernelGGL(merge_bwd<512>, grid, dim3(256), 0, st, m);
  else hipLaunchKernelGGL(merge_bwd<256>, grid, dim3(256), 0, st, m);
  return check_launch("mixed_merge_backward");
}

// ---- RoPE of the chunk's queries and keys (batched_engine.py:156, register.apply_rope) ----------------------------
// y = x cos + rotate_half(x) sin for x [B,H,n,d] bf16 and cos / sin [B,n,d] (fp32, or bf16) broadcast over the heads,
// as torch evaluates it: with fp32 tables each product and the sum rounded to fp32 (x - rotate_half(x) is exact),
// then the result rounded to bf16; with bf16 tables every operation rounded to bf16. The backward gives
// dx = bf16(bf16(dy cos) + rotate_half^T(bf16(dy sin))) for dy fp32, autograd's order of roundings for a bf16 x.
// One thread per 8 columns of each half of a row (8 threads per 128-wide row); up to two tensors per launch.
namespace hla {
namespace {

struct RopeParams {
  int count, B, H, n, d;
  const void* x[2];  // forward: bf16 x; backward: fp32 dy
  int64_t x_sb[2], x_sh[2], x_si[2];
  uint16_t* y[2];    // bf16
  int64_t y_sb[2], y_sh[2], y_si[2];
  const void* cos;
  const void* sin;
  int64_t c_sb, c_si;
  bool trig_bf16;
};

// 8 consecutive table values from column `off` (fp32, or bf16 with trig_bf16)
__device__ __forceinline__ void rope_trig8(const RopeParams& a, const void* t, int64_t off, float (&v)[8]) {
  if (a.trig_bf16) {
    const u32x4 w = ld16(static_cast<const uint16_t*>(t) + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = lo_bf(w[e]);
      v[2 * e + 1] = hi_bf(w[e]);
    }
  } else {
    const floatx4 x0 = *reinterpret_cast<const floatx4*>(static_cast<const float*>(t) + off);
    const floatx4 x1 = *reinterpret_cast<const floatx4*>(static_cast<const float*>(t) + off + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = x0[e];
      v[4 + e] = x1[e];
    }
  }
}

__device__ __forceinline__ float rope_mul(float a, float b, bool bf) { return bf ? rbf(__fmul_rn(a, b)) : __fmul_rn(a, b); }
__device__ __forceinline__ float rope_add(float a, float b, bool bf) { return bf ? rbf(__fadd_rn(a, b)) : __fadd_rn(a, b); }

// One thread per 8 columns of each half of a row: columns j .. j+7 and j+h2 .. j+h2+7 (16-byte accesses).
template <bool kBackward>
__global__ __launch_bounds__(256) void rope_rows(RopeParams a) {
  const int per_row = a.d / 16;
  const int64_t rows = (int64_t)a.B * a.H * a.n;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t r = gid / per_row;
  if (r >= rows * a.count) return;
  const int tsel = (int)(r / rows);
  const int64_t rr = r % rows;
  const int64_t b = rr / ((int64_t)a.H * a.n), h = (rr / a.n) % a.H, i = rr % a.n;
  const int h2 = a.d / 2, j = 8 * (int)(gid % per_row);
  const int64_t co = b * a.c_sb + i * a.c_si;
  float cl[8], ch[8], sl[8], sh[8];
  rope_trig8(a, a.cos, co + j, cl);
  rope_trig8(a, a.cos, co + j + h2, ch);
  rope_trig8(a, a.sin, co + j, sl);
  rope_trig8(a, a.sin, co + j + h2, sh);
  const bool bf = a.trig_bf16;
  const int64_t xo = b * a.x_sb[tsel] + h * a.x_sh[tsel] + i * a.x_si[tsel];
  float x1[8], x2[8];
  if constexpr (kBackward) {
    const float* xr = static_cast<const float*>(a.x[tsel]) + xo;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const floatx4 u = *reinterpret_cast<const floatx4*>(xr + j + 4 * half);
      const floatx4 v = *reinterpret_cast<const floatx4*>(xr + j + h2 + 4 * half);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x1[4 * half + e] = u[e];
        x2[4 * half + e] = v[e];
      }
    }
  } else {
    const uint16_t* xr = static_cast<const uint16_t*>(a.x[tsel]) + xo;
    const u32x4 u = ld16(xr + j), v = ld16(xr + j + h2);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x1[2 * e] = lo_bf(u[e]);
      x1[2 * e + 1] = hi_bf(u[e]);
      x2[2 * e] = lo_bf(v[e]);
      x2[2 * e + 1] = hi_bf(v[e]);
    }
  }
  float y1[8], y2[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if constexpr (kBackward) {  // dx1 = dy1 cos1 + dy2 sin2, dx2 = dy2 cos2 - dy1 sin1, each product rounded to bf16
      y1[e] = __fadd_rn(rbf(__fmul_rn(x1[e], cl[e])), rbf(__fmul_rn(x2[e], sh[e])));
      y2[e] = __fadd_rn(rbf(__fmul_rn(x2[e], ch[e])), -rbf(__fmul_rn(x1[e], sl[e])));
    } else {  // y1 = x1 cos1 - x2 sin1, y2 = x2 cos2 + x1 sin2
      y1[e] = rope_add(rope_mul(x1[e], cl[e], bf), rope_mul(-x2[e], sl[e], bf), bf);
      y2[e] = rope_add(rope_mul(x2[e], ch[e], bf), rope_mul(x1[e], sh[e], bf), bf);
    }
  }
  uint16_t* yr = a.y[tsel] + b * a.y_sb[tsel] + h * a.y_sh[tsel] + i * a.y_si[tsel];
  st16(yr + j, u32x4{pack2(y1[0], y1[1]), pack2(y1[2], y1[3]), pack2(y1[4], y1[5]), pack2(y1[6], y1[7])});
  st16(yr + j + h2, u32x4{pack2(y2[0], y2[1]), pack2(y2[2], y2[3]), pack2(y2[4], y2[5]), pack2(y2[6], y2[7])});
}

int rope_launch(bool backward, int32_t count, const void* const* x, const int64_t* x_strides, void* const* y,
                const int64_t* y_strides, int32_t batch, int32_t heads, int32_t chunk, int32_t head_dim,
                const void* cos, const void* sin, int64_t c_sb, int64_t c_si, int32_t trig_bf16, void* stream) {
  HLA_REQUIRE(count >= 1 && count <= 2 && batch >= 0 && heads >= 1 && chunk >= 0, HLA_S6_EINVAL,
              "rope_rows: bad tensor count, batch, head or chunk count");
  HLA_REQUIRE(head_dim >= 16 && head_dim % 16 == 0, HLA_S6_EUNSUPPORTED,
              "rope_rows: head_dim %d not a multiple of 16", head_dim);
  const int64_t rows = (int64_t)batch * heads * chunk;
  if (rows == 0) return HLA_S6_OK;
  HLA_REQUIRE(x && x_strides && y && y_strides && cos && sin, HLA_S6_EINVAL, "rope_rows: null pointer argument");
  HLA_REQUIRE(((uintptr_t)cos | (uintptr_t)sin) % 16 == 0 && c_sb % 8 == 0 && c_si % 8 == 0, HLA_S6_EINVAL,
              "rope_rows: cos / sin rows must be 16-byte aligned with a unit last stride");
  RopeParams p = {};
  p.count = count;
  p.B = batch;
  p.H = heads;
  p.n = chunk;
  p.d = head_dim;
  for (int t = 0; t < count; ++t) {
    HLA_REQUIRE(x[t] && y[t], HLA_S6_EINVAL, "rope_rows: null tensor %d", t);
    HLA_REQUIRE((uintptr_t)x[t] % 16 == 0 && (uintptr_t)y[t] % 16 == 0, HLA_S6_EINVAL,
                "rope_rows: tensor %d must be 16-byte aligned", t);
    for (int k = 0; k < 3; ++k)
      HLA_REQUIRE(x_strides[3 * t + k] % 8 == 0 && y_strides[3 * t + k] % 8 == 0, HLA_S6_EINVAL,
                  "rope_rows: strides of tensor %d must be multiples of 8 (16-byte rows)", t);
    p.x[t] = x[t];
    p.x_sb[t] = x_strides[3 * t];
    p.x_sh[t] = x_strides[3 * t + 1];
    p.x_si[t] = x_strides[3 * t + 2];
    p.y[t] = static_cast<uint16_t*>(y[t]);
    p.y_sb[t] = y_strides[3 * t];
    p.y_sh[t] = y_strides[3 * t + 1];
    p.y_si[t] = y_strides[3 * t + 2];
  }
  p.cos = cos;
  p.sin = sin;
  p.c_sb = c_sb;
  p.c_si = c_si;
  p.trig_bf16 = trig_bf16 != 0;
  const int64_t threads = rows * count * (head_dim / 16);
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (backward) hipLaunchKernelGGL(rope_rows<true>, grid, dim3(256), 0, as_stream(stream), p);
  else hipLaunchKernelGGL(rope_rows<false>, grid, dim3(256), 0, as_stream(stream), p);
  return check_launch("rope_rows");
}

}  // namespace
}  // namespace hla

extern "C" int hla_s6_rope_rows_forward(int32_t count, const void* const* x, const int64_t* x_strides, void* const* y,
                                        const int64_t* y_strides, int32_t batch, int32_t num_heads, int32_t chunk,
                                        int32_t head_dim, const void* cos, const void* sin, int64_t c_sb,
                                        int64_t c_si, int32_t trig_bf16, void* stream) {
  return hla::rope_launch(false, count, x, x_strides, y, y_strides, batch, num_heads, chunk, head_dim, cos, sin, c_sb,
                          c_si, trig_bf16, stream);
}

extern "C" int hla_s6_rope_rows_backward(int32_t count, const float* const* dy, const int64_t* dy_strides,
                                         void* const* dx, const int64_t* dx_strides, int32_t batch, int32_t num_heads,
                                         int32_t chunk, int32_t head_dim, const void* cos, const void* sin,
                                         int64_t c_sb, int64_t c_si, int32_t trig_bf16, void* stream) {
  return hla::rope_launch(true, count, reinterpret_cast<const void* const*>(dy), dy_strides, dx, dx_strides, batch,
                          num_heads, chunk, head_dim, cos, sin, c_sb, c_si, trig_bf16, stream);
}
