// Step metadata, block-table expansion, latent RoPE, LSE merges and slot-mapped row stores.
#include "common.h"

namespace hla {
namespace {

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline unsigned blocks_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

// ---- a1: token -> request, valid, ctx, ctx_latent, history --------------------------------------
__global__ void step_metadata_kernel(const int32_t* qsl, int R, const int32_t* seq_lens, int T, int window,
                                     int64_t* treq, uint8_t* valid, uint8_t* invalid, int32_t* ctx, int32_t* ctx_lat,
                                     int32_t* hist) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (hist && i < R) hist[i] = max(seq_lens[i] - (qsl[i + 1] - qsl[i]), 0);
  if (i >= T) return;
  int lo = 1, hi = R + 1;  // first r in [1, R] with qsl[r] > i
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (qsl[mid] > i) hi = mid;
    else lo = mid + 1;
  }
  const int req = min(lo - 1, R - 1);
  const bool v = i < qsl[R];
  if (treq) treq[i] = req;
  if (valid) valid[i] = v ? 1 : 0;
  if (invalid) invalid[i] = v ? 0 : 1;
  if (ctx || ctx_lat) {
    const int c = v ? max(seq_lens[req] - (qsl[req + 1] - qsl[req]), 0) : 0;
    if (ctx) ctx[i] = c;
    if (ctx_lat) ctx_lat[i] = window ? max(c - window, 0) : c;
  }
}

__global__ void gather_rows_kernel(const int32_t* table, int64_t ts, int cols, const int64_t* treq, int32_t* out,
                                   int64_t os) {
  const int t = blockIdx.x;
  const int32_t* src = table + treq[t] * ts;
  int32_t* dst = out + (int64_t)t * os;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) dst[c] = src[c];
}

// ---- a2/a3: in-place neox latent RoPE, torch bf16 op order ---------------------------------------
__global__ void latent_rope_kernel(uint16_t* x, int T, int H, int half, int64_t st, int64_t sh, const int64_t* pos,
                                   const uint16_t* table, int rows, int64_t ts) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)T * H * half;
  if (idx >= total) return;
  const int c = (int)(idx % half);
  const int64_t th = idx / half;
  const int h = (int)(th % H), t = (int)(th / H);
  uint16_t* row = x + (int64_t)t * st + (int64_t)h * sh;
  const uint16_t* tr = table + min(max(pos[t], (int64_t)0), (int64_t)rows - 1) * ts;
  const float x1 = bf2f(row[c]), x2 = bf2f(row[c + half]);
  const float cs = bf2f(tr[c]), sn = bf2f(tr[half + c]);
  row[c] = f2bf(rbf(x1 * cs) - rbf(x2 * sn));
  row[c + half] = f2bf(rbf(x2 * cs) + rbf(x1 * sn));
}

// ---- a8: LSE merges ------------------------------------------------------------------------------
__device__ __forceinline__ float nan_to_num(float v) {
  if (v != v) return 0.f;
  if (v == INFINITY) return 3.4028234663852886e38f;
  if (v == -INFINITY) return -3.4028234663852886e38f;
  return v;
}

__global__ void merge_kernel(const uint16_t* oa, int64_t a_st, int64_t a_sh, const float* lse_a, const uint16_t* ob,
                             int64_t b_st, int64_t b_sh, const float* lse_b, const uint8_t* invalid, int T, int H,
                             int D, int mode, uint16_t* out, int64_t o_st, int64_t o_sh, float* lse_out) {
  const int per_row = D / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)T * H * per_row) return;
  const int c = (int)(idx % per_row) * 8;
  const int64_t rowi = idx / per_row;
  const int h = (int)(rowi % H), t = (int)(rowi / H);
  float la = lse_a[(int64_t)h * T + t], lb = lse_b[(int64_t)h * T + t];
  if (mode == 0) {
    if (la == INFINITY) la = -INFINITY;
    if (lb == INFINITY) lb = -INFINITY;
  }
  float peak = fmaxf(la, lb);
  if (isinf(peak)) peak = 0.f;
  float wa = expf(la - peak), wb = expf(lb - peak);
  const float total = wa + wb;
  if (total > 0.f) {
    wa = wa / total;
    wb = wb / total;
  } else {
    wa = 0.f;
    wb = 0.f;
  }
  uint16_t* op = out + (int64_t)t * o_st + (int64_t)h * o_sh + c;
  if (mode == 0 && invalid && invalid[t]) {
    st16(op, u32x4{0u, 0u, 0u, 0u});
    return;
  }
  const u32x4 va = ld16(oa + (int64_t)t * a_st + (int64_t)h * a_sh + c);
  const u32x4 vb = ld16(ob + (int64_t)t * b_st + (int64_t)h * b_sh + c);
  u32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float a0 = lo_bf(va[e]), a1 = hi_bf(va[e]), b0 = lo_bf(vb[e]), b1 = hi_bf(vb[e]);
    if (mode == 1) {
      a0 = nan_to_num(a0);
      a1 = nan_to_num(a1);
      b0 = nan_to_num(b0);
      b1 = nan_to_num(b1);
    }
    r[e] = pack2(a0 * wa + b0 * wb, a1 * wa + b1 * wb);
  }
  st16(op, r);
  if (mode == 1 && lse_out && c == 0) lse_out[(int64_t)h * T + t] = peak + logf(total);
}

// ---- a10: slot mapping and row store --------------------------------------------------------------
__global__ void slot_mapping_kernel(const int32_t* bt, int64_t bs_stride, int cols, const int64_t* treq,
                                    const uint8_t* valid, const int64_t* pos, int T, int block, int64_t* slots) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const int64_t p = pos[t];
  if (!valid[t] || p < 0 || p / block >= cols) {
    slots[t] = -1;
    return;
  }
  slots[t] = (int64_t)bt[treq[t] * bs_stride + p / block] * block + p % block;
}

template <bool VEC>
__global__ void store_rows_kernel(const uint16_t* key, int64_t k_st, const uint16_t* value, int64_t v_st, int width,
                                  const int64_t* slots, uint16_t* cache, int64_t page_stride, int64_t row_stride,
                                  int block, int64_t num_blocks) {
  const int t = blockIdx.x;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_blocks * block) return;
  uint16_t* dst = cache + (slot / block) * page_stride + (slot % block) * row_stride;
  const uint16_t* ks = key + (int64_t)t * k_st;
  const uint16_t* vs = value + (int64_t)t * v_st;
  if (VEC) {  // 16-byte pieces
    const int chunks = width / 8;
    for (int c = threadIdx.x; c < 2 * chunks; c += blockDim.x) {
      const bool is_v = c >= chunks;
      const int cc = (is_v ? c - chunks : c) * 8;
      st16(dst + (is_v ? width : 0) + cc, ld16((is_v ? vs : ks) + cc));
    }
  } else {
    for (int c = threadIdx.x; c < 2 * width; c += blockDim.x) dst[c] = c < width ? ks[c] : vs[c - width];
  }
}

}  // namespace
}  // namespace hla

using namespace hla;

extern "C" int hla_s6_step_metadata(const int32_t* query_start_loc, int32_t num_reqs, const int32_t* seq_lens,
                                    int32_t num_tokens, int32_t window, int64_t* token_requests, uint8_t* valid,
                                    uint8_t* invalid, int32_t* ctx, int32_t* ctx_latent, int32_t* history,
                                    void* stream) {
  HLA_REQUIRE(num_reqs >= 1 && num_tokens >= 0 && window >= 0, HLA_S6_EINVAL,
              "step_metadata: need num_reqs >= 1, num_tokens >= 0, window >= 0");
  HLA_REQUIRE(query_start_loc, HLA_S6_EINVAL, "step_metadata: null query_start_loc");
  HLA_REQUIRE(seq_lens || !(ctx || ctx_latent || history), HLA_S6_EINVAL,
              "step_metadata: ctx, ctx_latent and history need seq_lens");
  const int n = max(num_tokens, num_reqs);
  hipLaunchKernelGGL(step_metadata_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream),
                     query_start_loc, num_reqs, seq_lens, num_tokens, window, token_requests, valid, invalid, ctx,
                     ctx_latent, history);
  return check_launch("step_metadata");
}

extern "C" int hla_s6_gather_block_table(const int32_t* table, int64_t table_stride, int32_t num_reqs, int32_t cols,
                                         const int64_t* token_requests, int32_t num_tokens, int32_t* out,
                                         int64_t out_stride, void* stream) {
  HLA_REQUIRE(num_tokens >= 0 && cols >= 0 && num_reqs >= 1, HLA_S6_EINVAL, "gather_block_table: bad sizes");
  if (num_tokens == 0 || cols == 0) return HLA_S6_OK;
  HLA_REQUIRE(table && token_requests && out, HLA_S6_EINVAL, "gather_block_table: null pointer");
  hipLaunchKernelGGL(gather_rows_kernel, dim3(num_tokens), dim3(cols < 256 ? 64 : 256), 0, as_stream(stream), table,
                     table_stride, cols, token_requests, out, out_stride);
  return check_launch("gather_block_table");
}

extern "C" int hla_s6_latent_rope(void* x, int32_t num_tokens, int32_t num_heads, int32_t width, int64_t stride_t,
                                  int64_t stride_h, const int64_t* positions, const void* table, int32_t table_rows,
                                  int64_t table_stride, void* stream) {
  HLA_REQUIRE(num_tokens >= 0 && num_heads >= 1 && width > 0 && width % 2 == 0, HLA_S6_EINVAL,
              "latent_rope: need an even width and positive head count");
  HLA_REQUIRE(table_rows > 0 && table_stride >= width, HLA_S6_EINVAL, "latent_rope: bad table geometry");
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(x && positions && table, HLA_S6_EINVAL, "latent_rope: null pointer");
  const int64_t total = (int64_t)num_tokens * num_heads * (width / 2);
  hipLaunchKernelGGL(latent_rope_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, as_stream(stream),
                     static_cast<uint16_t*>(x), num_tokens, num_heads, width / 2, stride_t, stride_h, positions,
                     static_cast<const uint16_t*>(table), table_rows, table_stride);
  return check_launch("latent_rope");
}

extern "C" int hla_s6_merge_states(const void* o_a, int64_t a_st, int64_t a_sh, const float* lse_a, const void* o_b,
                                   int64_t b_st, int64_t b_sh, const float* lse_b, const uint8_t* invalid,
                                   int32_t num_tokens, int32_t num_heads, int32_t head_dim, int32_t mode, void* out,
                                   int64_t o_st, int64_t o_sh, float* lse_out, void* stream) {
  HLA_REQUIRE(mode == 0 || mode == 1, HLA_S6_EINVAL, "merge_states: mode must be 0 or 1");
  HLA_REQUIRE(mode == 1 || lse_out == nullptr, HLA_S6_EINVAL, "merge_states: lse_out is only written by mode 1");
  HLA_REQUIRE(num_tokens >= 0 && num_heads >= 1 && head_dim > 0 && head_dim % 8 == 0, HLA_S6_EUNSUPPORTED,
              "merge_states: head_dim must be a multiple of 8");
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(o_a && o_b && lse_a && lse_b && out, HLA_S6_EINVAL, "merge_states: null pointer");
  HLA_REQUIRE(aligned16(o_a) && aligned16(o_b) && aligned16(out) && a_st % 8 == 0 && a_sh % 8 == 0 && b_st % 8 == 0 &&
                  b_sh % 8 == 0 && o_st % 8 == 0 && o_sh % 8 == 0,
              HLA_S6_EINVAL, "merge_states: rows must be 16-byte aligned");
  const int64_t total = (int64_t)num_tokens * num_heads * (head_dim / 8);
  hipLaunchKernelGGL(merge_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, as_stream(stream),
                     static_cast<const uint16_t*>(o_a), a_st, a_sh, lse_a, static_cast<const uint16_t*>(o_b), b_st,
                     b_sh, lse_b, invalid, num_tokens, num_heads, head_dim, mode, static_cast<uint16_t*>(out), o_st,
                     o_sh, lse_out);
  return check_launch("merge_states");
}

extern "C" int hla_s6_slot_mapping(const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                                   const int64_t* token_requests, const uint8_t* valid, const int64_t* positions,
                                   int32_t num_tokens, int32_t block_size, int64_t* slots, void* stream) {
  HLA_REQUIRE(num_tokens >= 0 && block_size > 0, HLA_S6_EINVAL, "slot_mapping: bad sizes");
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(block_table && token_requests && valid && positions && slots, HLA_S6_EINVAL,
              "slot_mapping: null pointer");
  hipLaunchKernelGGL(slot_mapping_kernel, dim3(blocks_for(num_tokens, 256)), dim3(256), 0, as_stream(stream),
                     block_table, bt_stride, bt_cols, token_requests, valid, positions, num_tokens, block_size, slots);
  return check_launch("slot_mapping");
}

extern "C" int hla_s6_store_rows(const void* key, int64_t k_st, const void* value, int64_t v_st, int32_t num_tokens,
                                 int32_t width, const int64_t* slots, void* cache, int64_t page_stride,
                                 int64_t row_stride, int32_t block_size, int64_t num_blocks, void* stream) {
  HLA_REQUIRE(num_tokens >= 0 && width > 0 && block_size > 0 && num_blocks >= 1, HLA_S6_EINVAL,
              "store_rows: bad width, block size or cache size");
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(key && value && slots && cache, HLA_S6_EINVAL, "store_rows: null pointer");
  const bool vec = width % 8 == 0 && aligned16(key) && aligned16(value) && aligned16(cache) && k_st % 8 == 0 &&
                   v_st % 8 == 0 && page_stride % 8 == 0 && row_stride % 8 == 0;
  const auto* k = static_cast<const uint16_t*>(key);
  const auto* v = static_cast<const uint16_t*>(value);
  auto* c = static_cast<uint16_t*>(cache);
  if (vec) {
    hipLaunchKernelGGL(store_rows_kernel<true>, dim3(num_tokens), dim3(128), 0, as_stream(stream), k, k_st, v, v_st,
                       width, slots, c, page_stride, row_stride, block_size, num_blocks);
  } else {
    hipLaunchKernelGGL(store_rows_kernel<false>, dim3(num_tokens), dim3(128), 0, as_stream(stream), k, k_st, v, v_st,
                       width, slots, c, page_stride, row_stride, block_size, num_blocks);
  }
  return check_launch("store_rows");
}
