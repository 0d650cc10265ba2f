// Exact (per-head K/V, head_dim 128) attention of one query row over a short key range, computed by one wave.
//
// The 64 lanes form 4 groups of 16; lane (group g, index i) holds head dims [8i, 8i+8). Keys are taken in
// batches of kExactBatch keys: every load of a batch (K and V rows, one 16-byte piece per lane) is issued
// before any arithmetic, so a W = 32 window plus the current token costs one memory round trip. Group g
// scores keys kb + 4*j + g; scores are reduced inside the 16-lane group and every group keeps its own
// online-softmax state, merged by LSE across the four groups at the end.
#pragma once

#include "common.h"

namespace hla {

constexpr int kExactDim = 128;
constexpr int kExactSteps = 9;                  // keys per group per batch
constexpr int kExactBatch = 4 * kExactSteps;    // 36 keys per batch

__device__ __forceinline__ float group_sum16(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  return v + __shfl_xor(v, 8);
}

// Source of key rows: a paged exact cache ([num_blocks, block, H, 2d] physical) or dense [T, H, d] tensors.
struct ExactSource {
  const uint16_t* k;
  const uint16_t* v;
  bool paged;
  // paged
  const int32_t* table_row;  // block-table row of the query
  int64_t page_stride, row_stride, head_stride, num_blocks;
  int block_size;
  // dense
  int64_t k_st, k_sh, v_st, v_sh;

  __device__ __forceinline__ void rows(int key, int h, int d0, const uint16_t*& kp, const uint16_t*& vp) const {
    if (paged) {
      const int64_t page = min(max((int64_t)table_row[key / block_size], (int64_t)0), num_blocks - 1);
      const int64_t off = page * page_stride + (int64_t)(key % block_size) * row_stride + (int64_t)h * head_stride + d0;
      kp = k + off;
      vp = v + off;
    } else {
      kp = k + (int64_t)key * k_st + (int64_t)h * k_sh + d0;
      vp = v + (int64_t)key * v_st + (int64_t)h * v_sh + d0;
    }
  }
};

// Softmax over keys [lo, hi) of head h for the query q (bf16 row of 128); writes o (bf16, 128) and the natural-log
// lse. Empty ranges give o = 0, lse = -inf. Must be called by all 64 lanes of a wave.
__device__ __forceinline__ void exact_row(const ExactSource& src, const uint16_t* q, float scale_log2, int lo, int hi,
                                          int h, int lane, uint16_t* out, float* lse_out) {
  const int grp = lane >> 4, d0 = (lane & 15) * 8;
  float qf[8];
  {
    const u32x4 qv = ld16(q + d0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qf[2 * e] = lo_bf(qv[e]) * scale_log2;
      qf[2 * e + 1] = hi_bf(qv[e]) * scale_log2;
    }
  }
  float m = -INFINITY, l = 0.f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;

  for (int kb = lo; kb < hi; kb += kExactBatch) {
    u32x4 kv[kExactSteps], vv[kExactSteps];
#pragma unroll
    for (int j = 0; j < kExactSteps; ++j) {
      const int key = kb + 4 * j + grp;
      kv[j] = u32x4{0u, 0u, 0u, 0u};
      vv[j] = u32x4{0u, 0u, 0u, 0u};
      if (key < hi) {
        const uint16_t *kp, *vp;
        src.rows(key, h, d0, kp, vp);
        kv[j] = ld16(kp);
        vv[j] = ld16(vp);
      }
    }
#pragma unroll
    for (int j = 0; j < kExactSteps; ++j) {
      const bool valid = kb + 4 * j + grp < hi;
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) dot += qf[2 * e] * lo_bf(kv[j][e]) + qf[2 * e + 1] * hi_bf(kv[j][e]);
      dot = group_sum16(dot);
      if (valid) {
        const float m_new = fmaxf(m, dot);
        const float alpha = fast_exp2(m - m_new);
        const float p = fast_exp2(dot - m_new);
        l = l * alpha + p;
        m = m_new;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[2 * e] = o[2 * e] * alpha + p * lo_bf(vv[j][e]);
          o[2 * e + 1] = o[2 * e + 1] * alpha + p * hi_bf(vv[j][e]);
        }
      }
    }
  }

  const float M = wave_max16x4(m);
  uint16_t* op = out + d0;
  if (M == -INFINITY) {
    if (grp == 0) st16(op, u32x4{0u, 0u, 0u, 0u});
    if (lane == 0) *lse_out = -INFINITY;
    return;
  }
  const float sc = (m == -INFINITY) ? 0.f : fast_exp2(m - M);
  const float L = wave_sum16x4(l * sc);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o[e] = wave_sum16x4(o[e] * sc);
  }
  if (grp == 0) {
    const float inv = 1.0f / L;
    st16(op, u32x4{pack2(o[0] * inv, o[1] * inv), pack2(o[2] * inv, o[3] * inv), pack2(o[4] * inv, o[5] * inv),
                   pack2(o[6] * inv, o[7] * inv)});
  }
  if (lane == 0) *lse_out = (M + log2f(L)) * kLn2;
}

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

// Decode-window key range of token t: query i of a request with Lq queries sits at p = seq_len - Lq + i and reads
// keys [max(0, p - window), p] (window_attention_fa semantics), or with chunk_start [max(0, seq_len - Lq - window), p]:
// the window's history rows before the chunk and the chunk's keys up to the query (the chunk attention and the
// window history of a prefill step in one range). Both are [seq_len - 1 - window, seq_len - 1] for Lq = 1. Returns
// false for padding tokens.
__device__ __forceinline__ bool decode_window_range(const int32_t* qsl, const int32_t* seq_lens, int R, int t,
                                                    int window, int& req, int& lo, int& hi, bool chunk_start = false,
                                                    const int64_t* token_requests = nullptr) {
  lo = hi = 0;
  req = 0;
  bool direct;
  if (token_requests) {  // the step's token -> request map: no search
    if (t >= qsl[R]) return false;
    req = (int)token_requests[t];
    direct = false;
  } else {
    // one query per request up to token t (a decode batch): token t is request t, found with two independent loads
    // instead of a dependent binary search
    direct = t < R && qsl[t] == t && qsl[t + 1] == t + 1;
    if (!direct) {
      if (t >= qsl[R]) return false;
      req = request_of(qsl, R, t);
    } else {
      req = t;
    }
  }
  const int lq = direct ? 1 : qsl[req + 1] - qsl[req];
  const int p = seq_lens[req] - lq + (direct ? 0 : t - qsl[req]);
  if (p >= 0) {
    lo = max(0, (chunk_start ? seq_lens[req] - lq : p) - window);
    hi = p + 1;
  }
  return true;
}

}  // namespace hla
