// Exact (per-head K/V) attention over short key ranges: the decode sliding window over the exact paged
// cache, the history-only window of prefill/mixed steps, and the causal current chunk. One wave per
// (token, head) running exact_row (exact.h).
#include "exact.h"

namespace hla {
namespace {

struct ExactParams {
  const uint16_t* q;
  int64_t q_st, q_sh;
  ExactSource src;
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

__global__ __launch_bounds__(256) void exact_attention(ExactParams a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pair = blockIdx.x * 4 + wave;
  if (pair >= a.T * a.H) return;
  const int t = pair / a.H, h = pair % a.H;
  int lo = 0, hi = 0;
  int64_t row = 0;
  if (a.mode == 0) {
    int req;
    decode_window_range(a.qsl, a.seq_lens, a.num_reqs, t, a.window, req, lo, hi);
    row = req;
  } else if (a.mode == 2) {
    if (t < a.qsl[a.num_reqs]) {
      lo = a.qsl[request_of(a.qsl, a.num_reqs, t)];
      hi = t + 1;
    }
  } else {
    const int c = a.ctx[t];
    lo = max(0, c - a.window);
    hi = c;
    row = a.bt_rows ? a.bt_rows[t] : (int64_t)t;
  }
  ExactSource src = a.src;
  if (src.paged) {
    hi = (int)min((int64_t)hi, (int64_t)a.bt_cols * src.block_size);  // keys the block table addresses
    src.table_row = a.bt + row * a.bt_stride;
  }
  exact_row(src, a.q + (int64_t)t * a.q_st + (int64_t)h * a.q_sh, a.scale_log2, lo, hi, h, lane,
            a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh, a.lse + (int64_t)h * a.T + t);
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
  HLA_REQUIRE(head_dim == kExactDim, HLA_S6_EUNSUPPORTED, "window_attention: head_dim %d (the kernel is built for 128)",
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
  p.src.k = static_cast<const uint16_t*>(k_cache);
  p.src.v = static_cast<const uint16_t*>(v_cache);
  p.src.paged = true;
  p.src.page_stride = page_stride;
  p.src.row_stride = row_stride;
  p.src.head_stride = head_stride;
  p.src.block_size = block_size;
  p.src.num_blocks = num_blocks;
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
  HLA_REQUIRE(head_dim == kExactDim, HLA_S6_EUNSUPPORTED, "chunk_attention: head_dim %d (the kernel is built for 128)",
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
  p.src.k = static_cast<const uint16_t*>(k);
  p.src.v = static_cast<const uint16_t*>(v);
  p.src.paged = false;
  p.src.k_st = k_st;
  p.src.k_sh = k_sh;
  p.src.v_st = v_st;
  p.src.v_sh = v_sh;
  p.src.block_size = 1;
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
