// Paged latent-history attention for the S6 MQA cache (16 query heads share one latent row).
//
// Kernel 1 (history_split): one workgroup per (token, KV split), 4 waves. Wave w owns the latent
// columns [w*R/4, (w+1)*R/4) of the query, of K and of V. Keys are walked in tiles of 16 rows (a
// tile never crosses a page since the page size is a multiple of 16):
//   * S^T[16 keys x 16 heads] = K . Q^T on v_mfma_f32_16x16x32_bf16. Each wave contracts its own
//     latent quarter: K rows are loaded straight into the MFMA A-operand layout (lane l: key l%16,
//     8 consecutive latent columns), Q^T is the B operand, held in registers for the whole row.
//     The four quarter partials are summed through LDS (one barrier per tile, double-buffered).
//   * online softmax in the exp2 domain on the 4 keys x 1 head each lane owns (cross-lane max/sum
//     over the 4 lane groups sharing a head);
//   * O^T[16 cols x 16 heads] += V^T . P^T on v_mfma_f32_16x16x16_bf16: P^T comes straight from the
//     softmax registers (the S^T output layout is the B-operand layout), V^T is read from a
//     wave-private LDS copy of the wave's V columns (transposing 16-bit reads).
//   * K/V loads of the next two tiles are in flight while a tile is computed.
// Each split writes its normalized partial output and natural-log LSE to the fp32 workspace
// (or, with a single split, the final bf16 output and LSE directly).
// Kernel 2 (history_combine): LSE reduction of the split partials into o [T,16,R] bf16, lse [16,T].
#include "common.h"

namespace hla {
namespace {

constexpr int kHeads = 16;
constexpr int kTile = 16;
constexpr int kThreads = 256;

struct HistoryParams {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t page_stride, row_stride;
  int block_size;
  int64_t num_blocks;
  const int32_t* bt;
  int64_t bt_stride;
  int bt_cols;
  const int64_t* bt_rows;
  const int32_t* ctx;
  float scale_log2;
  int num_splits;
  int T;
  float* ws_o;    // [T][S][16][R]
  float* ws_lse;  // [T][S][16]
  uint16_t* out;
  int64_t o_st, o_sh;
  float* lse;  // [16][T]
};

template <int R>
struct Geo {
  static constexpr int QW = R / 4;          // latent columns per wave
  static constexpr int KI = QW / 32;        // 16-byte K pieces per lane per tile (= MFMA k-steps)
  static constexpr int VC = QW / 32;        // 16-byte V chunks per lane per tile
  static constexpr int NT = QW / 16;        // 16-column O^T tiles per wave
  static constexpr int CPR = QW / 8;        // 16-byte chunks per V row (wave's columns)
  static constexpr int VS = QW + 8;         // LDS row stride of the V copy, in bf16
  static constexpr int VBUF = kTile * VS;   // one wave buffer, in bf16
};

template <int R>
struct TileRegs {
  u32x4 k[Geo<R>::KI];
  u32x4 v[Geo<R>::VC];
};

template <int R>
__device__ __forceinline__ void load_tile(const HistoryParams& a, const int32_t* btr, int n, int j, int col0,
                                          int lane, TileRegs<R>& r) {
  using G = Geo<R>;
  const int key0 = j * kTile;
  const int64_t page = min(max((int64_t)btr[key0 / a.block_size], (int64_t)0), a.num_blocks - 1);
  const int64_t base = page * a.page_stride + (int64_t)(key0 % a.block_size) * a.row_stride + col0;
  const int hq = lane & 15, g = lane >> 4;
  const bool kval = key0 + hq < n;
  const uint16_t* kp = a.k + base + (int64_t)hq * a.row_stride + 8 * g;
#pragma unroll
  for (int i = 0; i < G::KI; ++i) r.k[i] = kval ? ld16(kp + 32 * i) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int it = 0; it < G::VC; ++it) {
    const int c = it * 64 + lane;
    const int key = c / G::CPR;
    const int cc = (c % G::CPR) * 8;
    r.v[it] = (key0 + key < n) ? ld16(a.v + base + (int64_t)key * a.row_stride + cc) : u32x4{0u, 0u, 0u, 0u};
  }
}

// Stage A: V -> wave-private LDS, quarter-latent S^T partial. Consumes the tile registers.
template <int R>
__device__ __forceinline__ floatx4 stage_a(const TileRegs<R>& r, const u32x4 (&qreg)[Geo<R>::KI], uint16_t* vs,
                                           int lane) {
  using G = Geo<R>;
#pragma unroll
  for (int it = 0; it < G::VC; ++it) {
    const int c = it * 64 + lane;
    st16(vs + (c / G::CPR) * G::VS + (c % G::CPR) * 8, r.v[it]);
  }
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < G::KI; ++i) acc = mfma16x16x32(r.k[i], qreg[i], acc);
  return acc;
}

// Stage B: exchange S partials, online softmax, O^T += V^T P^T.
template <int R>
__device__ __forceinline__ void stage_b(floatx4 sacc, floatx4* sx, const uint16_t* vs, int key0, int n, float scale_log2,
                                        int wave, int lane, floatx4 (&oacc)[Geo<R>::NT], float& m, float& l) {
  using G = Geo<R>;
  sx[wave * 64 + lane] = sacc;
  __syncthreads();
  const floatx4 s = ((sx[lane] + sx[64 + lane]) + sx[128 + lane]) + sx[192 + lane];
  const int hq = lane & 15, g = lane >> 4;
  const int kb = key0 + 4 * g;
  float sc[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) sc[r] = (kb + r < n) ? s[r] * scale_log2 : -INFINITY;
  float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
  mx = wave_max16x4(mx);
  const float m_new = fmaxf(m, mx);
  const float alpha = fast_exp2(m - m_new);
  float p[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) p[r] = fast_exp2(sc[r] - m_new);
  const float ps = wave_sum16x4((p[0] + p[1]) + (p[2] + p[3]));
  l = l * alpha + ps;
  m = m_new;
  short4v pb;
#pragma unroll
  for (int r = 0; r < 4; ++r) pb[r] = (short)f2bf(p[r]);
#pragma unroll
  for (int nt = 0; nt < G::NT; ++nt) {
    short4v va;
#pragma unroll
    for (int e = 0; e < 4; ++e) va[e] = (short)vs[(4 * g + e) * G::VS + 16 * nt + hq];
    oacc[nt] = oacc[nt] * alpha;
    oacc[nt] = mfma16x16x16(va, pb, oacc[nt]);
  }
}

template <int R>
__global__ __launch_bounds__(kThreads) void history_split(HistoryParams a) {
  using G = Geo<R>;
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[4][2][G::VBUF];
  __shared__ floatx4 s_lds[2][4 * 64];
  __shared__ int red_lds[kThreads / 64];

  const int t = blockIdx.x, s = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int hq = lane & 15, g = lane >> 4;
  const int S = a.num_splits;
  const int64_t cap = (int64_t)a.bt_cols * a.block_size;  // keys the block table can address
  const int n = (int)min((int64_t)a.ctx[t], cap);
  const int tiles = (n + kTile - 1) / kTile;

  // Split partition: a fixed tile chunk for every row of the step, sized from the longest row, so that
  // rows of a ragged batch get split counts proportional to their length and every split has equal work.
  int chunk = tiles;
  if (S > 1) {
    int mx = 0;
    for (int i = tid; i < a.T; i += kThreads) mx = max(mx, (int)min((int64_t)a.ctx[i], cap));
    for (int off = 32; off > 0; off >>= 1) mx = max(mx, __shfl_xor(mx, off));
    if (lane == 0) red_lds[wave] = mx;
    __syncthreads();
    mx = max(max(red_lds[0], red_lds[1]), max(red_lds[2], red_lds[3]));
    const int max_tiles = (mx + kTile - 1) / kTile;
    chunk = (max_tiles + S - 1) / S;
  }
  const int j_begin = s * chunk;
  const int j_end = min(tiles, j_begin + chunk);
  const int col0 = wave * G::QW;

  if (j_begin >= j_end) {  // nothing to read in this split (uniform over the workgroup)
    if (S == 1) {
      uint16_t* op = a.out + (int64_t)t * a.o_st + (int64_t)hq * a.o_sh + col0 + 4 * g;
#pragma unroll
      for (int nt = 0; nt < G::NT; ++nt) *reinterpret_cast<uint2*>(op + 16 * nt) = uint2{0u, 0u};
      if (wave == 0 && g == 0) a.lse[(int64_t)hq * a.T + t] = -INFINITY;
    } else if (wave == 0 && g == 0) {
      a.ws_lse[((int64_t)t * S + s) * kHeads + hq] = -INFINITY;
    }
    return;
  }

  const int32_t* btr = a.bt + (a.bt_rows ? a.bt_rows[t] : (int64_t)t) * a.bt_stride;

  u32x4 qreg[G::KI];
  {
    const uint16_t* qp = a.q + (int64_t)t * a.q_st + (int64_t)hq * a.q_sh + col0 + 8 * g;
#pragma unroll
    for (int i = 0; i < G::KI; ++i) qreg[i] = ld16(qp + 32 * i);
  }

  floatx4 oacc[G::NT];
#pragma unroll
  for (int nt = 0; nt < G::NT; ++nt) oacc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  uint16_t* vs0 = v_lds[wave][0];
  uint16_t* vs1 = v_lds[wave][1];
  TileRegs<R> ra, rb;
  load_tile<R>(a, btr, n, j_begin, col0, lane, ra);
  if (j_begin + 1 < j_end) load_tile<R>(a, btr, n, j_begin + 1, col0, lane, rb);
  for (int j = j_begin; j < j_end; j += 2) {
    floatx4 sa = stage_a<R>(ra, qreg, vs0, lane);
    if (j + 2 < j_end) load_tile<R>(a, btr, n, j + 2, col0, lane, ra);
    stage_b<R>(sa, s_lds[0], vs0, j * kTile, n, a.scale_log2, wave, lane, oacc, m, l);
    if (j + 1 < j_end) {
      floatx4 sb = stage_a<R>(rb, qreg, vs1, lane);
      if (j + 3 < j_end) load_tile<R>(a, btr, n, j + 3, col0, lane, rb);
      stage_b<R>(sb, s_lds[1], vs1, (j + 1) * kTile, n, a.scale_log2, wave, lane, oacc, m, l);
    }
  }

  const float inv = 1.0f / l;
  const float lse = (m + log2f(l)) * kLn2;
  if (S == 1) {
    uint16_t* op = a.out + (int64_t)t * a.o_st + (int64_t)hq * a.o_sh + col0 + 4 * g;
#pragma unroll
    for (int nt = 0; nt < G::NT; ++nt) {
      const floatx4 o = oacc[nt] * inv;
      *reinterpret_cast<uint2*>(op + 16 * nt) = uint2{pack2(o[0], o[1]), pack2(o[2], o[3])};
    }
    if (wave == 0 && g == 0) a.lse[(int64_t)hq * a.T + t] = lse;
  } else {
    const int64_t row = ((int64_t)t * S + s) * kHeads + hq;
    float* wp = a.ws_o + row * R + col0 + 4 * g;
#pragma unroll
    for (int nt = 0; nt < G::NT; ++nt) *reinterpret_cast<floatx4*>(wp + 16 * nt) = oacc[nt] * inv;
    if (wave == 0 && g == 0) a.ws_lse[row] = lse;
  }
}

// One workgroup per (token, head); thread i owns output columns [4i, 4i+4).
template <int R>
__global__ __launch_bounds__(R / 4) void history_combine(const float* ws_o, const float* ws_lse, int S, int T,
                                                         uint16_t* out, int64_t o_st, int64_t o_sh, float* lse) {
  const int t = blockIdx.x, h = blockIdx.y, i = threadIdx.x;
  const float* ls = ws_lse + (int64_t)t * S * kHeads + h;
  float mx = -INFINITY;
  for (int s = 0; s < S; ++s) mx = fmaxf(mx, ls[(int64_t)s * kHeads]);
  uint16_t* op = out + (int64_t)t * o_st + (int64_t)h * o_sh + 4 * i;
  if (mx == -INFINITY) {
    *reinterpret_cast<uint2*>(op) = uint2{0u, 0u};
    if (i == 0) lse[(int64_t)h * T + t] = -INFINITY;
    return;
  }
  float den = 0.f;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < S; ++s) {
    const float ls_s = ls[(int64_t)s * kHeads];
    if (ls_s == -INFINITY) continue;
    const float w = __expf(ls_s - mx);
    den += w;
    const floatx4 o = *reinterpret_cast<const floatx4*>(ws_o + (((int64_t)t * S + s) * kHeads + h) * R + 4 * i);
    acc += o * w;
  }
  acc = acc * (1.0f / den);
  *reinterpret_cast<uint2*>(op) = uint2{pack2(acc[0], acc[1]), pack2(acc[2], acc[3])};
  if (i == 0) lse[(int64_t)h * T + t] = mx + logf(den);
}

template <int R>
int launch(const HistoryParams& p, hipStream_t stream) {
  dim3 grid(p.T, p.num_splits);
  hipLaunchKernelGGL(history_split<R>, grid, dim3(kThreads), 0, stream, p);
  int rc = check_launch("history_split");
  if (rc != HLA_S6_OK || p.num_splits == 1) return rc;
  hipLaunchKernelGGL(history_combine<R>, dim3(p.T, kHeads), dim3(R / 4), 0, stream, p.ws_o, p.ws_lse, p.num_splits,
                     p.T, p.out, p.o_st, p.o_sh, p.lse);
  return check_launch("history_combine");
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace hla

extern "C" int hla_s6_history_attention(const void* q, int32_t num_tokens, int32_t num_heads, int32_t width,
                                        int64_t q_st, int64_t q_sh, const void* k_cache, const void* v_cache,
                                        int64_t page_stride, int64_t row_stride, int32_t block_size,
                                        int64_t num_blocks, const int32_t* block_table, int64_t bt_stride,
                                        int32_t bt_cols, const int64_t* bt_rows,
                                        const int32_t* ctx, float scale, int32_t num_splits, float* workspace,
                                        int64_t workspace_floats, void* out, int64_t o_st, int64_t o_sh, float* lse,
                                        void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_tokens >= 0, HLA_S6_EINVAL, "history_attention: negative token count");
  HLA_REQUIRE(num_heads == kHeads, HLA_S6_EUNSUPPORTED, "history_attention: %d query heads (the kernel is built for 16)",
              num_heads);
  HLA_REQUIRE(width == 128 || width == 256 || width == 512 || width == 1024, HLA_S6_EUNSUPPORTED,
              "history_attention: latent width %d not in {128, 256, 512, 1024}", width);
  HLA_REQUIRE(block_size > 0 && block_size % kTile == 0, HLA_S6_EUNSUPPORTED,
              "history_attention: block size %d is not a positive multiple of 16", block_size);
  HLA_REQUIRE(num_splits >= 1, HLA_S6_EINVAL, "history_attention: num_kv_splits must be >= 1");
  HLA_REQUIRE(num_blocks >= 1 && bt_cols >= 0, HLA_S6_EINVAL, "history_attention: empty cache or bad table width");
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(q && k_cache && v_cache && block_table && ctx && out && lse, HLA_S6_EINVAL,
              "history_attention: null pointer argument");
  HLA_REQUIRE(aligned16(q) && q_st % 8 == 0 && q_sh % 8 == 0, HLA_S6_EINVAL,
              "history_attention: q needs 16-byte aligned rows (unit last stride, strides multiple of 8)");
  HLA_REQUIRE(aligned16(k_cache) && aligned16(v_cache) && page_stride % 8 == 0 && row_stride % 8 == 0, HLA_S6_EINVAL,
              "history_attention: cache rows must be 16-byte aligned (strides multiple of 8 elements)");
  HLA_REQUIRE((reinterpret_cast<uintptr_t>(out) & 7u) == 0 && o_st % 4 == 0 && o_sh % 4 == 0, HLA_S6_EINVAL,
              "history_attention: output rows must be 8-byte aligned");
  if (num_splits > 1) {
    const int64_t need = (int64_t)num_tokens * num_splits * kHeads * (width + 1);
    HLA_REQUIRE(workspace != nullptr && workspace_floats >= need, HLA_S6_EWORKSPACE,
                "S6 workspace overflow: need %lld floats, have %lld", (long long)need, (long long)workspace_floats);
    HLA_REQUIRE(aligned16(workspace), HLA_S6_EINVAL, "history_attention: workspace must be 16-byte aligned");
  }
  HLA_REQUIRE(num_splits <= 65535, HLA_S6_EINVAL, "history_attention: too many splits");
  HistoryParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.q_st = q_st;
  p.q_sh = q_sh;
  p.k = static_cast<const uint16_t*>(k_cache);
  p.v = static_cast<const uint16_t*>(v_cache);
  p.page_stride = page_stride;
  p.row_stride = row_stride;
  p.block_size = block_size;
  p.num_blocks = num_blocks;
  p.bt = block_table;
  p.bt_stride = bt_stride;
  p.bt_cols = bt_cols;
  p.bt_rows = bt_rows;
  p.ctx = ctx;
  p.scale_log2 = scale * kLog2e;
  p.num_splits = num_splits;
  p.T = num_tokens;
  p.ws_o = workspace;
  p.ws_lse = workspace ? workspace + (int64_t)num_tokens * num_splits * kHeads * width : nullptr;
  p.out = static_cast<uint16_t*>(out);
  p.o_st = o_st;
  p.o_sh = o_sh;
  p.lse = lse;
  hipStream_t st = as_stream(stream);
  switch (width) {
    case 128: return launch<128>(p, st);
    case 256: return launch<256>(p, st);
    case 512: return launch<512>(p, st);
    default: return launch<1024>(p, st);
  }
}
