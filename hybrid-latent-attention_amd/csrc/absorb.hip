// Batched per-head projections out[t, h, :] = x[t, h, :] @ w[h] (A_t absorption and B_t projection).
//
// One workgroup computes 64 tokens x 64 output columns of one head: 4 waves, each 16 tokens x 4 column
// tiles of 16, on v_mfma_f32_16x16x32_bf16. Every global load of the workgroup is issued before the first
// barrier: the whole weight slab w[h, :, 64 columns] (K x 128 bytes) and each wave's x rows (the A operand,
// k contiguous, straight into MFMA layout). The slab goes to LDS row-major with 16-byte stores (rows 72 elements
// apart: conflict-free) and the B operand (8 consecutive k of one column) comes back by two ds_read_b64_tr_b16.
// Epilogues:
//   * STORE: bf16 result;
//   * ROPE: latent RoPE of the bf16-rounded product (fused latent_query); the four column tiles are then
//     {c, c+16, c+N/2, c+N/2+16}, so every lane holds both rotation partners of its outputs.
#include "common.h"

namespace hla {
namespace {

enum Epilogue { kStore = 0, kRope = 1 };

struct AbsorbParams {
  const uint16_t* x;
  int64_t x_st, x_sh;
  const uint16_t* w;
  int64_t w_sh, w_sk;
  uint16_t* out;
  int64_t o_st, o_sh;
  int T, N;
  // ROPE
  const int64_t* pos;
  const uint16_t* table;
  int table_rows;
  int64_t table_stride;
};

template <int K, int EPI>
__global__ __launch_bounds__(256) void absorb_kernel(AbsorbParams a) {
  constexpr int LS = 72;                // LDS row stride of the slab (one k per row, 64 columns + 8), bf16
  constexpr int CH = K / 32;            // 16-byte slab pieces per thread (K * 8 pieces / 256 threads)
  extern __shared__ __attribute__((aligned(16))) uint16_t wt[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, g = lane >> 4;
  const int h = blockIdx.y;
  const int t0 = blockIdx.z * 64 + wave * 16;
  int ct[4];
  if (EPI == kRope) {
    const int half = a.N / 2, base = blockIdx.x * 32;
    ct[0] = base;
    ct[1] = base + 16;
    ct[2] = base + half;
    ct[3] = base + half + 16;
  } else {
    const int base = blockIdx.x * 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) ct[i] = base + 16 * i;
  }

  // issue every global load first
  const uint16_t* wh = a.w + (int64_t)h * a.w_sh;
  u32x4 slab[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = i * 256 + tid;
    const int kr = c >> 3, cchunk = c & 7;
    slab[i] = ld16(wh + (int64_t)kr * a.w_sk + ct[cchunk >> 1] + (cchunk & 1) * 8);
  }
  const int ta = t0 + l16;
  u32x4 xa[CH];
  {
    const uint16_t* xrow = a.x + (int64_t)ta * a.x_st + (int64_t)h * a.x_sh + 8 * g;
#pragma unroll
    for (int i = 0; i < CH; ++i) xa[i] = ta < a.T ? ld16(xrow + 32 * i) : u32x4{0u, 0u, 0u, 0u};
  }
  // RoPE epilogue operands (positions, then the table rows) in flight with the slab
  float rcos[4][2], rsin[4][2];
  if (EPI == kRope) {
    const int half = a.N / 2;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = min(t0 + 4 * g + r, a.T - 1);
      const uint16_t* tr = a.table + min(max(a.pos[t], (int64_t)0), (int64_t)a.table_rows - 1) * a.table_stride;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        rcos[r][i] = bf2f(tr[ct[i] + l16]);
        rsin[r][i] = bf2f(tr[half + ct[i] + l16]);
      }
    }
  }
  // the slab into LDS row-major: wt[k][local column], local column 16 i + j is column ct[i] + j
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = i * 256 + tid;
    const int kr = c >> 3, cchunk = c & 7;
    st16(wt + kr * LS + cchunk * 8, slab[i]);
  }
  __syncthreads();

  floatx4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  // B operand of lane (g, l16): wt[32 kk + 8 g + e][16 i + l16], e < 8 (lane j of a 16-lane group addresses row
  // 32 kk + 8 g + j / 4, columns 16 i + 4 (j % 4) ..; the transposing read hands lane l16 its column)
  const uint16_t* tp = wt + (8 * g + (l16 >> 2)) * LS + 4 * (l16 & 3);
#pragma unroll
  for (int kk = 0; kk < CH; ++kk) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t* p = tp + 32 * kk * LS + 16 * i;
      const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)p);
      const short4v hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)(p + 4 * LS));
      acc[i] = mfma16x16x32(xa[kk], join_tr(lo, hi), acc[i]);
    }
  }

  // lane holds out[t0 + 4g + r][ct[i] + l16]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + 4 * g + r;
    if (t >= a.T) continue;
    uint16_t* orow = a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh;
    if (EPI == kRope) {
      const int half = a.N / 2;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = ct[i] + l16;
        const float x1 = rbf(acc[i][r]), x2 = rbf(acc[i + 2][r]);
        const float cs = rcos[r][i], sn = rsin[r][i];
        orow[c] = f2bf(rbf(x1 * cs) - rbf(x2 * sn));
        orow[c + half] = f2bf(rbf(x2 * cs) + rbf(x1 * sn));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) orow[ct[i] + l16] = f2bf(acc[i][r]);
    }
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int EPI>
int launch_k(const AbsorbParams& p, int K, int H, hipStream_t st) {
  const dim3 grid(p.N / 64, H, (unsigned)((p.T + 63) / 64));
  switch (K) {
#define HLA_ABSORB_CASE(KK)                                                                             \
  case KK: {                                                                                            \
    constexpr int lds = KK * 72 * 2;                                                                    \
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&absorb_kernel<KK, EPI>), \
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds); \
    if (attr != hipSuccess) return fail(HLA_S6_ELAUNCH, "absorb: LDS size %d rejected", lds);          \
    hipLaunchKernelGGL((absorb_kernel<KK, EPI>), grid, dim3(256), lds, st, p);                          \
    break;                                                                                              \
  }
    HLA_ABSORB_CASE(128)
    HLA_ABSORB_CASE(256)
    HLA_ABSORB_CASE(512)
    HLA_ABSORB_CASE(1024)
#undef HLA_ABSORB_CASE
    default:
      return fail(HLA_S6_EUNSUPPORTED, "absorb: k_dim %d not in {128, 256, 512, 1024}", K);
  }
  return check_launch("absorb");
}

int check_common(const void* x, int32_t num_tokens, int32_t num_heads, int32_t k_dim, int64_t x_st, int64_t x_sh,
                 const void* w, int64_t w_sh, int64_t w_sk, int32_t n_dim, const void* out) {
  HLA_REQUIRE(num_tokens >= 0 && num_heads >= 1 && num_heads <= 65535, HLA_S6_EINVAL, "absorb: bad token/head count");
  HLA_REQUIRE((k_dim == 128 || k_dim == 256 || k_dim == 512 || k_dim == 1024) && n_dim > 0 && n_dim % 64 == 0,
              HLA_S6_EUNSUPPORTED, "absorb: need k_dim in {128, 256, 512, 1024} and n_dim %% 64 == 0 (got %d, %d)",
              k_dim, n_dim);
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(x && w && out, HLA_S6_EINVAL, "absorb: null pointer");
  HLA_REQUIRE(aligned16(x) && x_st % 8 == 0 && x_sh % 8 == 0, HLA_S6_EINVAL,
              "absorb: x rows must be 16-byte aligned with a unit last stride");
  HLA_REQUIRE(aligned16(w) && w_sh % 8 == 0 && w_sk % 8 == 0, HLA_S6_EINVAL,
              "absorb: weight rows must be 16-byte aligned with a unit last stride");
  return HLA_S6_OK;
}

}  // namespace

}  // namespace hla

extern "C" int hla_s6_absorb(const void* x, int32_t num_tokens, int32_t num_heads, int32_t k_dim, int64_t x_st,
                             int64_t x_sh, const void* w, int64_t w_sh, int64_t w_sk, int32_t n_dim, void* out,
                             int64_t o_st, int64_t o_sh, const int64_t* positions, const void* rope_table,
                             int32_t table_rows, int64_t table_stride, void* stream) {
  using namespace hla;
  int rc = check_common(x, num_tokens, num_heads, k_dim, x_st, x_sh, w, w_sh, w_sk, n_dim, out);
  if (rc != HLA_S6_OK || num_tokens == 0) return rc;
  if (rope_table) {
    HLA_REQUIRE(positions != nullptr && table_rows > 0 && table_stride >= n_dim, HLA_S6_EINVAL,
                "absorb: RoPE epilogue needs positions and a [rows, n_dim] table");
  }
  AbsorbParams p = {};
  p.x = static_cast<const uint16_t*>(x);
  p.x_st = x_st;
  p.x_sh = x_sh;
  p.w = static_cast<const uint16_t*>(w);
  p.w_sh = w_sh;
  p.w_sk = w_sk;
  p.out = static_cast<uint16_t*>(out);
  p.o_st = o_st;
  p.o_sh = o_sh;
  p.T = num_tokens;
  p.N = n_dim;
  p.pos = positions;
  p.table = static_cast<const uint16_t*>(rope_table);
  p.table_rows = table_rows;
  p.table_stride = table_stride;
  hipStream_t st = as_stream(stream);
  return rope_table ? launch_k<kRope>(p, k_dim, num_heads, st) : launch_k<kStore>(p, k_dim, num_heads, st);
}
