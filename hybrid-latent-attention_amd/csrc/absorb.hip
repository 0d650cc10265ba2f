// Batched per-head projections out[t, h, :] = x[t, h, :] @ w[h] (A_t absorption and B_t projection).
//
// One workgroup computes 64 tokens x 64 output columns of one head: 4 waves, each 16 tokens x
// 4 column tiles of 16, on v_mfma_f32_16x16x32_bf16. x rows feed the A operand straight from global
// memory (k contiguous); the weight slab w[h, k-chunk, 64 columns] is staged in LDS transposed
// (column-major) so the B operand is one 16-byte LDS read per lane. With the latent RoPE epilogue the
// four column tiles are {c, c+16, c+N/2, c+N/2+16}: every lane then holds both rotation partners of its
// outputs and the rotation is applied in registers before the store.
#include "common.h"

namespace hla {
namespace {

constexpr int kKc = 128;  // k rows staged per LDS chunk
constexpr int kLdsStride = kKc + 8;

struct AbsorbParams {
  const uint16_t* x;
  int64_t x_st, x_sh;
  const uint16_t* w;
  int64_t w_sh, w_sk;
  uint16_t* out;
  int64_t o_st, o_sh;
  int T, K, N;
  const int64_t* pos;
  const uint16_t* table;
  int table_rows;
  int64_t table_stride;
};

template <bool ROPE>
__global__ __launch_bounds__(256) void absorb_kernel(AbsorbParams a) {
  __shared__ __attribute__((aligned(16))) uint16_t wt[64 * kLdsStride];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, g = lane >> 4;
  const int h = blockIdx.y;
  const int t0 = blockIdx.z * 64 + wave * 16;
  int ct[4];
  if (ROPE) {
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
  floatx4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int ta = t0 + l16;  // token row this lane feeds into the A operand
  const uint16_t* xrow = a.x + (int64_t)ta * a.x_st + (int64_t)h * a.x_sh + 8 * g;
  const uint16_t* wh = a.w + (int64_t)h * a.w_sh;

  for (int k0 = 0; k0 < a.K; k0 += kKc) {
    const int kc = min(kKc, a.K - k0);
    // stage w[h, k0:k0+kc, tiles] transposed: wt[col][k]
    for (int c = tid; c < kc * 8; c += 256) {
      const int kr = c >> 3, cchunk = c & 7;
      const int tile = cchunk >> 1, cin = (cchunk & 1) * 8;
      const u32x4 val = ld16(wh + (int64_t)(k0 + kr) * a.w_sk + ct[tile] + cin);
      uint16_t* dst = wt + (tile * 16 + cin) * kLdsStride + kr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dst[(2 * e) * kLdsStride] = (uint16_t)(val[e] & 0xffffu);
        dst[(2 * e + 1) * kLdsStride] = (uint16_t)(val[e] >> 16);
      }
    }
    __syncthreads();
    for (int kk = 0; kk < kc; kk += 32) {
      const u32x4 av = ta < a.T ? ld16(xrow + k0 + kk) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 bv = *reinterpret_cast<const u32x4*>(wt + (i * 16 + l16) * kLdsStride + kk + 8 * g);
        acc[i] = mfma16x16x32(av, bv, acc[i]);
      }
    }
    __syncthreads();
  }

  // lane holds out[t0 + 4g + r][ct[i] + l16]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + 4 * g + r;
    if (t >= a.T) continue;
    uint16_t* orow = a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh;
    if (ROPE) {
      const int half = a.N / 2;
      const uint16_t* tr = a.table + min(max(a.pos[t], (int64_t)0), (int64_t)a.table_rows - 1) * a.table_stride;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = ct[i] + l16;
        const float x1 = rbf(acc[i][r]), x2 = rbf(acc[i + 2][r]);
        const float cs = bf2f(tr[c]), sn = bf2f(tr[half + c]);
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

}  // namespace
}  // namespace hla

extern "C" int hla_s6_absorb(const void* x, int32_t num_tokens, int32_t num_heads, int32_t k_dim, int64_t x_st,
                             int64_t x_sh, const void* w, int64_t w_sh, int64_t w_sk, int32_t n_dim, void* out,
                             int64_t o_st, int64_t o_sh, const int64_t* positions, const void* rope_table,
                             int32_t table_rows, int64_t table_stride, void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_tokens >= 0 && num_heads >= 1 && num_heads <= 65535, HLA_S6_EINVAL, "absorb: bad token/head count");
  HLA_REQUIRE(k_dim > 0 && k_dim % 32 == 0 && n_dim > 0 && n_dim % 64 == 0, HLA_S6_EUNSUPPORTED,
              "absorb: need k_dim %% 32 == 0 and n_dim %% 64 == 0 (got %d, %d)", k_dim, n_dim);
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(x && w && out, HLA_S6_EINVAL, "absorb: null pointer");
  HLA_REQUIRE(aligned16(x) && x_st % 8 == 0 && x_sh % 8 == 0, HLA_S6_EINVAL,
              "absorb: x rows must be 16-byte aligned with a unit last stride");
  HLA_REQUIRE(aligned16(w) && w_sh % 8 == 0 && w_sk % 8 == 0, HLA_S6_EINVAL,
              "absorb: weight rows must be 16-byte aligned with a unit last stride");
  if (rope_table) {
    HLA_REQUIRE(positions != nullptr && table_rows > 0 && table_stride >= n_dim, HLA_S6_EINVAL,
                "absorb: RoPE epilogue needs positions and a [rows, n_dim] table");
  }
  AbsorbParams p;
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
  p.K = k_dim;
  p.N = n_dim;
  p.pos = positions;
  p.table = static_cast<const uint16_t*>(rope_table);
  p.table_rows = table_rows;
  p.table_stride = table_stride;
  const unsigned tiles_t = (unsigned)((num_tokens + 63) / 64);
  hipStream_t st = as_stream(stream);
  if (rope_table) {
    hipLaunchKernelGGL(absorb_kernel<true>, dim3(n_dim / 64, num_heads, tiles_t), dim3(256), 0, st, p);
  } else {
    hipLaunchKernelGGL(absorb_kernel<false>, dim3(n_dim / 64, num_heads, tiles_t), dim3(256), 0, st, p);
  }
  return check_launch("absorb");
}
