// Exact (per-head K/V) attention over short key ranges: the decode sliding window over the exact paged
// cache, the history-only window of prefill/mixed steps, and the causal current chunk.
//
// One wave per (token, head). The 64 lanes form 4 groups of 16; a group takes one key per step and
// each lane holds 8 of the 128 head dims, so a key row (K or V, 256 bytes) is one coalesced 16-byte
// load per lane. Scores are reduced inside the 16-lane group; every group keeps its own online
// softmax state (max, sum, 8 output dims) and the four groups are merged by LSE at the end.
#include "common.h"

namespace hla {
namespace {

constexpr int kDim = 128;

struct ExactParams {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  // paged source (window): page/row/head strides; dense source (chunk): token/head strides
  int64_t page_stride, row_stride, head_stride;
  int64_t k_st, k_sh, v_st, v_sh;
  int block_size;
  int64_t num_blocks;
  const int32_t* bt;
  int64_t bt_stride;
  int bt_cols;
  const int64_t* bt_rows;
  int mode;  // 0: decode window, 1: history window, 2: causal chunk
  const int32_t* qsl;
  const int32_t* seq_lens;
  int num_reqs;
  const int32_t* ctx;
  int window;
  float scale_log2;
  int T, H;
  uint16_t* out;
  int64_t o_st, o_sh;
  float* lse;
};

// Request index of token t: searchsorted(qsl[1:], t, right=True) clamped to num_reqs - 1.
__device__ __forceinline__ int request_of(const int32_t* qsl, int R, int t) {
  int lo = 1, hi = R + 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (qsl[mid] > t) hi = mid;
    else lo = mid + 1;
  }
  return min(lo - 1, R - 1);
}

__device__ __forceinline__ float group_sum16(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  return v + __shfl_xor(v, 8);
}

__global__ __launch_bounds__(256) void exact_attention(ExactParams a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pair = blockIdx.x * 4 + wave;
  if (pair >= a.T * a.H) return;
  const int t = pair / a.H, h = pair % a.H;
  const int grp = lane >> 4, d0 = (lane & 15) * 8;

  int lo = 0, hi = 0;
  int64_t row = 0;
  if (a.mode == 0 || a.mode == 2) {
    const int R = a.num_reqs;
    if (t < a.qsl[R]) {
      const int req = request_of(a.qsl, R, t);
      if (a.mode == 0) {
        const int lq = a.qsl[req + 1] - a.qsl[req];
        const int p = a.seq_lens[req] - lq + (t - a.qsl[req]);
        if (p >= 0) {
          lo = max(0, p - a.window);
          hi = p + 1;
        }
        row = req;
      } else {
        lo = a.qsl[req];
        hi = t + 1;
      }
    }
  } else {
    const int c = a.ctx[t];
    lo = max(0, c - a.window);
    hi = c;
    row = a.bt_rows ? a.bt_rows[t] : (int64_t)t;
  }

  if (a.mode != 2) hi = (int)min((int64_t)hi, (int64_t)a.bt_cols * a.block_size);  // keys the table addresses

  float qf[8];
  {
    const u32x4 qv = ld16(a.q + (int64_t)t * a.q_st + (int64_t)h * a.q_sh + d0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qf[2 * e] = lo_bf(qv[e]) * a.scale_log2;
      qf[2 * e + 1] = hi_bf(qv[e]) * a.scale_log2;
    }
  }
  float m = -INFINITY, l = 0.f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;

  const int32_t* btr = a.bt ? a.bt + row * a.bt_stride : nullptr;
  for (int kb = lo; kb < hi; kb += 4) {
    const int key = kb + grp;
    const bool valid = key < hi;
    u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
    if (valid) {
      const uint16_t *kp, *vp;
      if (a.mode == 2) {
        kp = a.k + (int64_t)key * a.k_st + (int64_t)h * a.k_sh + d0;
        vp = a.v + (int64_t)key * a.v_st + (int64_t)h * a.v_sh + d0;
      } else {
        const int64_t page = min(max((int64_t)btr[key / a.block_size], (int64_t)0), a.num_blocks - 1);
        const int64_t off = page * a.page_stride +
                            (int64_t)(key % a.block_size) * a.row_stride + (int64_t)h * a.head_stride + d0;
        kp = a.k + off;
        vp = a.v + off;
      }
      kv = ld16(kp);
      vv = ld16(vp);
    }
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) dot += qf[2 * e] * lo_bf(kv[e]) + qf[2 * e + 1] * hi_bf(kv[e]);
    dot = group_sum16(dot);
    if (valid) {
      const float m_new = fmaxf(m, dot);
      const float alpha = fast_exp2(m - m_new);
      const float p = fast_exp2(dot - m_new);
      l = l * alpha + p;
      m = m_new;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[2 * e] = o[2 * e] * alpha + p * lo_bf(vv[e]);
        o[2 * e + 1] = o[2 * e + 1] * alpha + p * hi_bf(vv[e]);
      }
    }
  }

  // LSE merge of the four group partials.
  float M = fmaxf(m, __shfl_xor(m, 16));
  M = fmaxf(M, __shfl_xor(M, 32));
  uint16_t* op = a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh + d0;
  if (M == -INFINITY) {
    if (grp == 0) st16(op, u32x4{0u, 0u, 0u, 0u});
    if (lane == 0) a.lse[(int64_t)h * a.T + t] = -INFINITY;
    return;
  }
  const float sc = (m == -INFINITY) ? 0.f : fast_exp2(m - M);
  float L = l * sc;
  L += __shfl_xor(L, 16);
  L += __shfl_xor(L, 32);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float x = o[e] * sc;
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    o[e] = x;
  }
  if (grp == 0) {
    const float inv = 1.0f / L;
    st16(op, u32x4{pack2(o[0] * inv, o[1] * inv), pack2(o[2] * inv, o[3] * inv), pack2(o[4] * inv, o[5] * inv),
                   pack2(o[6] * inv, o[7] * inv)});
  }
  if (lane == 0) a.lse[(int64_t)h * a.T + t] = (M + log2f(L)) * kLn2;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_exact(const ExactParams& p, hipStream_t stream, const char* what) {
  const int64_t pairs = (int64_t)p.T * p.H;
  HLA_REQUIRE(pairs <= (int64_t)1 << 31, HLA_S6_EINVAL, "%s: too many rows", what);
  hipLaunchKernelGGL(exact_attention, dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, stream, p);
  return check_launch(what);
}

}  // namespace
}  // namespace hla

extern "C" int hla_s6_window_attention(const void* q, int32_t num_tokens, int32_t num_heads, int32_t head_dim,
                                       int64_t q_st, int64_t q_sh, const void* k_cache, const void* v_cache,
                                       int64_t page_stride, int64_t row_stride, int64_t head_stride,
                                       int32_t block_size, int64_t num_blocks, const int32_t* block_table,
                                       int64_t bt_stride, int32_t bt_cols, const int64_t* bt_rows, int32_t mode,
                                       const int32_t* query_start_loc,
                                       const int32_t* seq_lens, int32_t num_reqs, const int32_t* ctx, int32_t window,
                                       float scale, void* out, int64_t o_st, int64_t o_sh, float* lse, void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_tokens >= 0 && num_heads > 0, HLA_S6_EINVAL, "window_attention: bad token/head count");
  HLA_REQUIRE(head_dim == kDim, HLA_S6_EUNSUPPORTED, "window_attention: head_dim %d (the kernel is built for 128)",
              head_dim);
  HLA_REQUIRE(mode == 0 || mode == 1, HLA_S6_EINVAL, "window_attention: mode must be 0 (decode) or 1 (history)");
  HLA_REQUIRE(window >= 0, HLA_S6_EINVAL, "window_attention: negative window");
  HLA_REQUIRE(block_size > 0 && num_blocks >= 1 && bt_cols >= 0, HLA_S6_EINVAL,
              "window_attention: bad block size, cache size or table width");
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(q && k_cache && v_cache && block_table && out && lse, HLA_S6_EINVAL, "window_attention: null pointer");
  HLA_REQUIRE(mode == 1 || (query_start_loc && seq_lens && num_reqs >= 1), HLA_S6_EINVAL,
              "window_attention: decode mode needs query_start_loc, seq_lens and num_reqs >= 1");
  HLA_REQUIRE(mode == 0 || ctx, HLA_S6_EINVAL, "window_attention: history mode needs ctx");
  HLA_REQUIRE(aligned16(q) && q_st % 8 == 0 && q_sh % 8 == 0 && aligned16(out) && o_st % 8 == 0 && o_sh % 8 == 0,
              HLA_S6_EINVAL, "window_attention: q/out rows must be 16-byte aligned");
  HLA_REQUIRE(aligned16(k_cache) && aligned16(v_cache) && page_stride % 8 == 0 && row_stride % 8 == 0 &&
                  head_stride % 8 == 0,
              HLA_S6_EINVAL, "window_attention: cache rows must be 16-byte aligned");
  ExactParams p = {};
  p.q = static_cast<const uint16_t*>(q);
  p.q_st = q_st;
  p.q_sh = q_sh;
  p.k = static_cast<const uint16_t*>(k_cache);
  p.v = static_cast<const uint16_t*>(v_cache);
  p.page_stride = page_stride;
  p.row_stride = row_stride;
  p.head_stride = head_stride;
  p.block_size = block_size;
  p.num_blocks = num_blocks;
  p.bt = block_table;
  p.bt_stride = bt_stride;
  p.bt_cols = bt_cols;
  p.bt_rows = bt_rows;
  p.mode = mode;
  p.qsl = query_start_loc;
  p.seq_lens = seq_lens;
  p.num_reqs = num_reqs;
  p.ctx = ctx;
  p.window = window;
  p.scale_log2 = scale * kLog2e;
  p.T = num_tokens;
  p.H = num_heads;
  p.out = static_cast<uint16_t*>(out);
  p.o_st = o_st;
  p.o_sh = o_sh;
  p.lse = lse;
  return launch_exact(p, as_stream(stream), "window_attention");
}

extern "C" int hla_s6_chunk_attention(const void* q, const void* k, const void* v, int32_t num_tokens,
                                      int32_t num_heads, int32_t head_dim, int64_t q_st, int64_t q_sh, int64_t k_st,
                                      int64_t k_sh, int64_t v_st, int64_t v_sh, const int32_t* query_start_loc,
                                      int32_t num_reqs, float scale, void* out, int64_t o_st, int64_t o_sh,
                                      float* lse, void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_tokens >= 0 && num_heads > 0, HLA_S6_EINVAL, "chunk_attention: bad token/head count");
  HLA_REQUIRE(head_dim == kDim, HLA_S6_EUNSUPPORTED, "chunk_attention: head_dim %d (the kernel is built for 128)",
              head_dim);
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(q && k && v && query_start_loc && num_reqs >= 1 && out && lse, HLA_S6_EINVAL,
              "chunk_attention: null pointer or no request");
  HLA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) && q_st % 8 == 0 && q_sh % 8 == 0 &&
                  k_st % 8 == 0 && k_sh % 8 == 0 && v_st % 8 == 0 && v_sh % 8 == 0 && o_st % 8 == 0 &&
                  o_sh % 8 == 0,
              HLA_S6_EINVAL, "chunk_attention: rows must be 16-byte aligned");
  ExactParams p = {};
  p.q = static_cast<const uint16_t*>(q);
  p.q_st = q_st;
  p.q_sh = q_sh;
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.k_st = k_st;
  p.k_sh = k_sh;
  p.v_st = v_st;
  p.v_sh = v_sh;
  p.block_size = 1;
  p.mode = 2;
  p.qsl = query_start_loc;
  p.num_reqs = num_reqs;
  p.scale_log2 = scale * kLog2e;
  p.T = num_tokens;
  p.H = num_heads;
  p.out = static_cast<uint16_t*>(out);
  p.o_st = o_st;
  p.o_sh = o_sh;
  p.lse = lse;
  return launch_exact(p, as_stream(stream), "chunk_attention");
}
