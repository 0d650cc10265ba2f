// Writer of the S6 terminal block: the per-loop candidate projection, its register accumulation and the
// committed-row store (hla/latent/register.py:45-61, hla/vllm_latent/s6_layer.py:124-147,
// hla/vllm_latent/ouro_latent.py:127-129), as one kernel.
//
//   u[t, n]   = bf16( sum_k h[t, k] * W[n, k] )                 (nn.Linear, bf16 output)
//   reg[t, n] = prev ? bf16(prev[t, n] + u[t, n]) : u[t, n]      (write_step: previous + update)
//   commit:     cache row slots[t] <- [RoPE_lat(reg[t, :w]) | reg[t, w:]]
//
// W is the nn.Linear weight [2w, hidden] (rows = output columns), so both MFMA operands are k-contiguous and
// come straight from global memory with 16-byte loads: lane l takes A = h[row l%16][k + 8(l/16) ..] and
// B = W[column l%16][k + 8(l/16) ..]. A workgroup computes 16 or 64 tokens x 16 output columns; its eight waves (four
// when hidden is not a multiple of 1024) take one slice of the hidden dimension each, with two batches of four
// v_mfma_f32_16x16x32_bf16 k steps in flight, so every operand byte of a decode step's workgroup is requested at
// once (the kernel is latency-bound at decode sizes); the per-wave fp32 partials are summed in LDS in a fixed order. A key-half tile holds 8 rotation pairs (columns c and c + w/2), so each thread of
// the epilogue has both partners of a RoPE pair; value-half tiles hold 16 consecutive columns.
#include "common.h"

namespace hla {
namespace {

struct WriterParams {
  const uint16_t* h;
  int64_t h_st;
  const uint16_t* w;
  int64_t w_st;
  const uint16_t* prev;
  int64_t prev_st;
  uint16_t* reg;
  int64_t reg_st;
  const int64_t* slots;
  const int64_t* pos;
  const uint16_t* table;
  int table_rows;
  int64_t table_stride;
  uint16_t* cache;
  int64_t page_stride, row_stride;
  int block;
  int64_t num_slots;
  int T, K, width;
};

// Output column of MFMA column j (0..15) of column tile x.
__device__ __forceinline__ int writer_col(int x, int j, int width) {
  const int key_tiles = width / 16;
  return x < key_tiles ? 8 * x + (j & 7) + (j >> 3) * (width / 2) : width + 16 * (x - key_tiles) + j;
}

template <int WAVES, int MT>
__global__ __launch_bounds__(WAVES * 64) void writer_kernel(WriterParams a) {
  __shared__ float red[WAVES][16 * MT][17];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, g = lane >> 4;
  const int x = blockIdx.x, t0 = blockIdx.y * 16 * MT;
  const int kw = a.K / WAVES, k0 = wave * kw;
  const int msub = min(MT, (a.T - t0 + 15) / 16);  // row tiles holding tokens (wave-uniform)

  const uint16_t* wrow = a.w + (int64_t)writer_col(x, l16, a.width) * a.w_st + k0 + 8 * g;
  const uint16_t* hrow[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) hrow[m] = a.h + (int64_t)min(t0 + 16 * m + l16, a.T - 1) * a.h_st + k0 + 8 * g;

  floatx4 acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
  // kw is a multiple of 128: batches of four 32-wide k steps, two batches in flight (the second batch's loads
  // are issued before the first batch's MFMAs)
  u32x4 b0[4], a0[4][MT], b1[4], a1[4][MT];
  auto issue = [&](u32x4(&bv)[4], u32x4(&av)[4][MT], int k) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bv[i] = ld16(wrow + k + 32 * i);
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if (m < msub) av[i][m] = ld16(hrow[m] + k + 32 * i);
    }
  };
  auto compute = [&](const u32x4(&bv)[4], const u32x4(&av)[4][MT]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if (m < msub) acc[m] = mfma16x16x32(av[i][m], bv[i], acc[m]);
  };
  issue(b0, a0, 0);
  for (int k = 0; k < kw; k += 256) {
    const bool second = k + 128 < kw;
    if (second) issue(b1, a1, k + 128);
    compute(b0, a0);
    if (k + 256 < kw) issue(b0, a0, k + 256);
    if (second) compute(b1, a1);
  }
  // lane holds D[4g + r][l16] of row tile m: token t0 + 16m + 4g + r, tile column l16
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][16 * m + 4 * g + r][l16] = acc[m][r];
  __syncthreads();

  // thread: token t0 + tid/4, tile columns q, q+4, q+8, q+12 (q = tid % 4): two rotation pairs in a key tile
  const int row = tid >> 2, q = tid & 3, t = t0 + row;
  if (row >= 16 * MT || t >= a.T) return;
  float v[4];
  int col[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = q + 4 * i;
    col[i] = writer_col(x, j, a.width);
    float sum = red[0][row][j];
#pragma unroll
    for (int v2 = 1; v2 < WAVES; ++v2) sum += red[v2][row][j];
    float u = rbf(sum);
    if (a.prev) u = rbf(bf2f(a.prev[(int64_t)t * a.prev_st + col[i]]) + u);
    v[i] = u;
    if (a.reg) a.reg[(int64_t)t * a.reg_st + col[i]] = f2bf(u);
  }
  if (!a.cache) return;
  const int64_t slot = a.slots[t];
  if (slot < 0 || slot >= a.num_slots) return;
  uint16_t* crow = a.cache + (slot / a.block) * a.page_stride + (slot % a.block) * a.row_stride;
  if (x < a.width / 16) {
    const int half = a.width / 2;
    const uint16_t* tr =
        a.table + min(max(a.pos[t], (int64_t)0), (int64_t)a.table_rows - 1) * a.table_stride;
#pragma unroll
    for (int p = 0; p < 2; ++p) {  // pair (col[p], col[p] + w/2) = (v[p], v[p + 2])
      const int c = col[p];
      const float cs = bf2f(tr[c]), sn = bf2f(tr[half + c]);
      const float x1 = v[p], x2 = v[p + 2];
      crow[c] = f2bf(rbf(x1 * cs) - rbf(x2 * sn));
      crow[c + half] = f2bf(rbf(x2 * cs) + rbf(x1 * sn));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) crow[col[i]] = f2bf(v[i]);
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace hla

extern "C" int hla_s6_write_rows(const void* h, int32_t num_tokens, int32_t hidden, int64_t h_st, const void* weight,
                                 int32_t width, int64_t w_st, const void* prev, int64_t prev_st, void* reg,
                                 int64_t reg_st, const int64_t* slots, const int64_t* positions,
                                 const void* rope_table, int32_t table_rows, int64_t table_stride, void* cache,
                                 int64_t page_stride, int64_t row_stride, int32_t block_size, int64_t num_blocks,
                                 void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_tokens >= 0 && num_tokens <= 65535 * 64, HLA_S6_EINVAL, "write_rows: bad token count %d",
              num_tokens);
  HLA_REQUIRE(width >= 16 && width % 16 == 0 && width <= 4096, HLA_S6_EUNSUPPORTED,
              "write_rows: width %d must be a multiple of 16 (at most 4096)", width);
  HLA_REQUIRE(hidden >= 512 && hidden % 512 == 0, HLA_S6_EUNSUPPORTED,
              "write_rows: hidden %d must be a positive multiple of 512", hidden);
  HLA_REQUIRE(reg || cache, HLA_S6_EINVAL, "write_rows: neither a register output nor a cache to commit to");
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(h && weight, HLA_S6_EINVAL, "write_rows: null input");
  HLA_REQUIRE(aligned16(h) && h_st % 8 == 0 && aligned16(weight) && w_st % 8 == 0 && h_st >= hidden &&
                  w_st >= hidden,
              HLA_S6_EINVAL, "write_rows: h and weight rows must be 16-byte aligned with a unit last stride");
  HLA_REQUIRE(!prev || prev_st >= 2 * width, HLA_S6_EINVAL, "write_rows: prev rows shorter than 2 * width");
  HLA_REQUIRE(!reg || reg_st >= 2 * width, HLA_S6_EINVAL, "write_rows: reg rows shorter than 2 * width");
  if (cache) {
    HLA_REQUIRE(slots && positions && rope_table && table_rows > 0 && table_stride >= width, HLA_S6_EINVAL,
                "write_rows: a commit needs slots, positions and a [rows, width] RoPE table");
    HLA_REQUIRE(block_size > 0 && num_blocks > 0 && row_stride >= 2 * width && page_stride >= row_stride,
                HLA_S6_EINVAL, "write_rows: bad cache geometry");
  }
  WriterParams p = {};
  p.h = static_cast<const uint16_t*>(h);
  p.h_st = h_st;
  p.w = static_cast<const uint16_t*>(weight);
  p.w_st = w_st;
  p.prev = static_cast<const uint16_t*>(prev);
  p.prev_st = prev_st;
  p.reg = static_cast<uint16_t*>(reg);
  p.reg_st = reg_st;
  p.slots = slots;
  p.pos = positions;
  p.table = static_cast<const uint16_t*>(rope_table);
  p.table_rows = table_rows;
  p.table_stride = table_stride;
  p.cache = static_cast<uint16_t*>(cache);
  p.page_stride = page_stride;
  p.row_stride = row_stride;
  p.block = block_size;
  p.num_slots = cache ? num_blocks * (int64_t)block_size : 0;
  p.T = num_tokens;
  p.K = hidden;
  p.width = width;
  // up to 128 tokens a workgroup takes 16 of them (more workgroups, fewer operand bytes per CU: the kernel is
  // latency-bound there); beyond, 64 (each weight tile is then read by fewer workgroups)
  const bool small = num_tokens <= 128;
  const int rows = small ? 16 : 64;
  const dim3 grid((unsigned)(width / 8), (unsigned)((num_tokens + rows - 1) / rows));
  hipStream_t st = as_stream(stream);
  if (hidden % 1024 == 0) {
    if (small)
      hipLaunchKernelGGL((writer_kernel<8, 1>), grid, dim3(512), 0, st, p);
    else
      hipLaunchKernelGGL((writer_kernel<8, 4>), grid, dim3(512), 0, st, p);
  } else {
    if (small)
      hipLaunchKernelGGL((writer_kernel<4, 1>), grid, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((writer_kernel<4, 4>), grid, dim3(256), 0, st, p);
  }
  return check_launch("write_rows");
}
