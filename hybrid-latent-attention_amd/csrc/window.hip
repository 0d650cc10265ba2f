// Exact (per-head K/V) attention: the decode sliding window over the exact paged cache and the history-only window
// of prefill/mixed steps (short key ranges: one wave per (token, head) running exact_row, exact.h), and the causal
// current chunk (chunk_mfma: sixteen tokens of one head per wave on MFMA).
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

// Causal attention inside each request's chunk: one workgroup of NW waves per (16 NW consecutive tokens, head), 16
// queries per wave. The tokens of a workgroup that belong to one request read that request's keys in tiles
// of 32 rows (16 with one wave), each tile loaded once for the workgroup (coalesced 16-byte pieces of K and of V,
// two tiles ahead in registers) and staged in LDS, double-buffered, one barrier per tile. Each wave then computes
//   S^T[16 keys x 16 queries] = K . Q^T per 16-key block on v_mfma_f32_16x16x32_bf16 (K rows from LDS as the A
//   operand, Q^T in registers), causal mask key <= query, online softmax per query column, and
//   O^T[128 x 16 queries] += V^T . P^T on v_mfma_f32_16x16x32_bf16 over the tile's 32 keys (16x16x16 over 16)
//   with V^T read from LDS by ds_read_b64_tr_b16,
// skipping the tiles wholly past its last query. Sharing the tiles over 64 queries instead of 16 cuts the L2 requests
// of the causal re-reads fourfold, which bound an earlier one-wave form that gathered K in 64-byte pieces; the
// single-wave blocks here copy whole coalesced tiles and run only where 64-token blocks would leave CUs idle.
struct ChunkParams {
  const uint16_t *q, *k, *v;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh;
  const int32_t* qsl;
  int num_reqs, T;
  float scale_log2;
  uint16_t* out;
  int64_t o_st, o_sh;
  float* lse;  // [H, T]
  // the exact window over the request's history rows [ctx - window, ctx), ctx = seq_len - query_len (chunk_window)
  ExactSource win;
  const int32_t* bt;  // per-request block table of the exact cache
  int64_t bt_stride;
  int bt_cols;
  const int32_t* seq_lens;
  int window;
  int nblk, heads;  // token blocks of kChunkQ and heads: the grid is nblk * heads workgroups
};

constexpr int kChunkVS = kExactDim + 16;    // LDS row stride of the V tile (conflict-free transposed reads)
constexpr int kChunkKS = kExactDim + 16;    // LDS row stride of the K tile (16-byte row reads: +8 conflicts, +16 not)
// Waves per workgroup, 16 queries each: 4 (the tiles shared by 64 queries), or 1 for steps of short requests whose
// grid of 64-token blocks leaves CUs idle (such a block would run several requests' passes one after another on one
// CU; 16-token blocks spread them).
template <int NW>
struct ChunkGeo {
  static constexpr int Q = 16 * NW;               // queries per workgroup
  static constexpr int TK = NW == 1 ? 16 : 32;    // keys per tile
  static constexpr int KB = TK / 16;              // 16-key blocks per tile
  static constexpr int P = TK * 16 / (64 * NW);   // 16-byte pieces of a tile per thread (K and V each)
  static constexpr int DEPTH = 2;                  // key tiles in flight (registers) per thread
};

template <bool kWin, int NW>
__global__ __launch_bounds__(64 * NW) void chunk_mfma(ChunkParams a) {
  using G = ChunkGeo<NW>;
  constexpr int kChunkQ = G::Q, kChunkDepth = G::DEPTH, P = G::P, TK = G::TK, KB = G::KB;
  __shared__ __attribute__((aligned(16))) uint16_t ks_l[2][TK * kChunkKS];
  __shared__ __attribute__((aligned(16))) uint16_t vs_l[2][TK * kChunkVS];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hq = lane & 15, g = lane >> 4;
  // Workgroup b runs on XCD b % 8 (workgroups are dealt to the XCDs round-robin). With a multiple of 8 heads, the
  // token blocks of head h all run on XCD h % 8, so the re-reads of a request's K/V rows by its token blocks hit
  // that XCD's L2; an XCD takes its heads' token blocks last to first (the longest causal rows first).
  const int b = blockIdx.x;
  int h, tb;
  if (a.heads % 8 == 0) {
    const int k = b >> 3;
    h = (b & 7) + 8 * (k / a.nblk);
    tb = a.nblk - 1 - k % a.nblk;
  } else {
    h = b / a.nblk;
    tb = a.nblk - 1 - b % a.nblk;
  }
  const int t_begin = tb * kChunkQ, t_end = min(t_begin + kChunkQ, a.T);
  const int valid_end = min(t_end, a.qsl[a.num_reqs]);
  for (int tp = t_begin; tp < t_end;) {
    int count, kb;
    if (tp >= valid_end) {  // padding tokens: o = 0, lse = -inf
      count = t_end - tp;
      kb = 0;
    } else {
      const int r = request_of(a.qsl, a.num_reqs, tp);
      count = min(valid_end, a.qsl[r + 1]) - tp;
      kb = a.qsl[r];
    }
    const bool live = tp < valid_end;
    const int ke = live ? tp + count : 0;  // keys [kb, ke): the request's tokens up to the pass's last query
    // window keys (history rows [w_lo, w_hi) of the exact cache, visible to every query of the request)
    int w_lo = 0, w_hi = 0;
    ExactSource src = a.win;
    if (kWin && live) {
      const int r = request_of(a.qsl, a.num_reqs, tp);
      w_hi = a.seq_lens[r] - (a.qsl[r + 1] - a.qsl[r]);
      w_lo = max(0, w_hi - a.window);
      w_hi = max(min(w_hi, a.bt_cols * src.block_size), w_lo);  // never negative: the chunk tiles follow
      src.table_row = a.bt + (int64_t)r * a.bt_stride;
    }
    // this wave's queries [qw, qw + cw) of the pass; a wave without one still takes part in the tile barriers
    const int qw = tp + 16 * wave, cw = max(0, min(count - 16 * wave, 16));
    const int last_q = qw + cw - 1;
    const int tq = cw > 0 ? qw + min(hq, cw - 1) : tp;  // query of this lane's column
    u32x4 qb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qb[i] = ld16(a.q + (int64_t)tq * a.q_st + (int64_t)h * a.q_sh + 32 * i + 8 * g);
    floatx4 oacc[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) oacc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;
    const int q_pos = qw + hq;  // this column's query token (keys <= q_pos are visible)
    const int nwt = (w_hi - w_lo + TK - 1) / TK;  // window tiles, taken before the chunk's (one online softmax)
    const int nct = ke > kb ? (ke - kb + TK - 1) / TK : 0;
    // this thread's pieces u of tile ti: piece c = tid + 64 NW u is row c / 16, bytes 16 * (c % 16) of K and of V
    // (rows past the tile's keys zeroed)
    auto load = [&](int ti, u32x4 (&kx)[P], u32x4 (&vx)[P]) {
      const bool wt = kWin && ti < nwt;
      const int k0 = wt ? w_lo + TK * ti : kb + TK * (ti - nwt);
      const int kend = wt ? w_hi : ke;
#pragma unroll
      for (int u = 0; u < P; ++u) {
        const int c = tid + 64 * NW * u;
        const int row = c >> 4, d0 = (c & 15) * 8, key = min(k0 + row, kend - 1);
        if (wt) {
          const uint16_t *kp, *vp;
          src.rows(key, h, d0, kp, vp);
          kx[u] = ld16(kp);
          vx[u] = ld16(vp);
        } else {
          kx[u] = ld16(a.k + (int64_t)key * a.k_st + (int64_t)h * a.k_sh + d0);
          vx[u] = ld16(a.v + (int64_t)key * a.v_st + (int64_t)h * a.v_sh + d0);
        }
        if (k0 + row >= kend) kx[u] = vx[u] = u32x4{0u, 0u, 0u, 0u};
      }
    };
    // this wave's part of tile ti from LDS: S^T, causal mask, online softmax, O^T += V^T P^T
    auto compute = [&](int ti, const uint16_t* ks, const uint16_t* vs) {
      const bool wt = kWin && ti < nwt;
      const int k0 = wt ? w_lo + TK * ti : kb + TK * (ti - nwt);
      const int kend = wt ? w_hi : ke;
      if (cw == 0 || (!wt && k0 > last_q)) return;  // no query of the wave sees a key of the tile (wave-uniform)
      floatx4 s[KB];
#pragma unroll
      for (int b2 = 0; b2 < KB; ++b2) {
        s[b2] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          s[b2] = mfma16x16x32(*reinterpret_cast<const u32x4*>(ks + (16 * b2 + hq) * kChunkKS + 32 * i + 8 * g), qb[i],
                               s[b2]);
      }
      float sc[KB][4];
      // wave-uniform: every key of the tile is visible to every query of the wave (a window tile inside the
      // window, or a chunk tile wholly before the wave's first query)
      const bool full = wt ? k0 + TK <= kend : k0 + TK <= ke && k0 + TK - 1 <= qw;
      if (full) {
#pragma unroll
        for (int b2 = 0; b2 < KB; ++b2)
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[b2][r] = hq < cw ? s[b2][r] * a.scale_log2 : -INFINITY;
      } else {
#pragma unroll
        for (int b2 = 0; b2 < KB; ++b2)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = k0 + 16 * b2 + 4 * g + r;
            const bool vis = wt ? key < kend : key < ke && key <= q_pos;
            sc[b2][r] = (vis && hq < cw) ? s[b2][r] * a.scale_log2 : -INFINITY;
          }
      }
      // (scores are finite or -inf: masked keys never reach a maximum); the running maximum is raised lazily, only
      // when a tile exceeds it by more than 2^8 (the exponentials stay below 2^8), which skips the rescale of the
      // accumulators on most tiles
      float mloc = max_nn(max_nn(sc[0][0], sc[0][1]), max_nn(sc[0][2], sc[0][3]));
#pragma unroll
      for (int b2 = 1; b2 < KB; ++b2)
        mloc = max_nn(mloc, max_nn(max_nn(sc[b2][0], sc[b2][1]), max_nn(sc[b2][2], sc[b2][3])));
      const float mx = wave_max16x4_nn(mloc);
      const bool raise = mx > m + 8.f;  // false while the column has no visible key (mx = -inf)
      if (__any(raise)) {
        const float m_new = raise ? mx : m;
        // 0 on the first raise (m = -inf); 1 in a column that does not raise, which may still have no visible key
        // (m = -inf: a column past the pass's queries)
        const float alpha = raise ? fast_exp2(m - m_new) : 1.f;
        l *= alpha;
        m = m_new;
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) oacc[nt] = oacc[nt] * alpha;
      }
      const float m_use = m == -INFINITY ? 0.f : m;
      float p[KB][4];
#pragma unroll
      for (int b2 = 0; b2 < KB; ++b2) {
#pragma unroll
        for (int r = 0; r < 4; ++r) p[b2][r] = fast_exp2(sc[b2][r] - m_use);
        l += (p[b2][0] + p[b2][1]) + (p[b2][2] + p[b2][3]);  // this lane's share of the column sum
      }
      if constexpr (KB == 1) {
        const uint32_t p01 = pack2_hw(p[0][0], p[0][1]), p23 = pack2_hw(p[0][2], p[0][3]);
        const short4v pb = {(short)(p01 & 0xffffu), (short)(p01 >> 16), (short)(p23 & 0xffffu), (short)(p23 >> 16)};
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          // lane (g, hq) of the A operand: V[4g + e][16nt + hq]; the transposing read takes row 4g + hq/4,
          // columns 16nt + 4(hq%4) .. +3 in each 16-lane group
          const uint16_t* vp = vs + (4 * g + (hq >> 2)) * kChunkVS + 16 * nt + 4 * (hq & 3);
          const short4v va =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)vp);
          oacc[nt] = mfma16x16x16(va, pb, oacc[nt]);
        }
      } else {
        // 32 keys on 16x16x32: k slot 8g + e holds key 4g + e of block 0 (e < 4) and of block 1 (e >= 4), for P^T
        // (the lane's own scores) and for V^T (two transposing reads, rows of block 0 then of block 1)
        const u32x4 pb = {pack2_hw(p[0][0], p[0][1]), pack2_hw(p[0][2], p[0][3]), pack2_hw(p[1][0], p[1][1]),
                          pack2_hw(p[1][2], p[1][3])};
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          const uint16_t* vp = vs + (4 * g + (hq >> 2)) * kChunkVS + 16 * nt + 4 * (hq & 3);
          const short4v lo =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)vp);
          const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) short4v*)(vp + 16 * kChunkVS));
          oacc[nt] = mfma16x16x32(join_tr(lo, hi), pb, oacc[nt]);
        }
      }
    };
    // kChunkDepth register sets in rotation: set d holds tiles d, d + kChunkDepth, ... and is reloaded as soon as
    // its tile is in LDS (compile-time indices: no register copies). LDS buffer ti % 2 is rewritten two tiles later,
    // after the barrier that every wave passes only once it has computed the tile before
    const int ntl = nwt + nct;
    u32x4 kx[kChunkDepth][P], vx[kChunkDepth][P];
#pragma unroll
    for (int d = 0; d < kChunkDepth; ++d)
      if (d < ntl) load(d, kx[d], vx[d]);
    for (int ti0 = 0; ti0 < ntl; ti0 += kChunkDepth) {
#pragma unroll
      for (int d = 0; d < kChunkDepth; ++d) {
        const int ti = ti0 + d;
        if (ti < ntl) {  // (uniform over the workgroup)
          uint16_t* ks = ks_l[ti & 1];
          uint16_t* vs = vs_l[ti & 1];
#pragma unroll
          for (int u = 0; u < P; ++u) {
            const int c = tid + 64 * NW * u;
            st16(ks + (c >> 4) * kChunkKS + (c & 15) * 8, kx[d][u]);
            st16(vs + (c >> 4) * kChunkVS + (c & 15) * 8, vx[d][u]);
          }
          if (ti + kChunkDepth < ntl) load(ti + kChunkDepth, kx[d], vx[d]);
          __syncthreads();
          compute(ti, ks, vs);
        }
      }
    }
    l = wave_sum16x4(l);
    if (hq < cw) {
      const int t = qw + hq;
      const bool any = l > 0.f;
      const float inv = any ? 1.0f / l : 0.f;
      uint16_t* op = a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh + 4 * g;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        const floatx4 o = oacc[nt] * inv;
        *reinterpret_cast<uint2*>(op + 16 * nt) = uint2{pack2(o[0], o[1]), pack2(o[2], o[3])};
      }
      if (g == 0) a.lse[(int64_t)h * a.T + t] = any ? (m + log2f(l)) * kLn2 : -INFINITY;
    }
    __syncthreads();  // the next pass rewrites the LDS tiles
    tp += count;
  }
}

// 16-token single-wave blocks when the requests average fewer than 64 tokens (a 64-token block would run several
// requests' passes one after another) and 64-token blocks x heads leave CUs idle; the 4-wave form otherwise
template <bool kWin>
void launch_chunk(ChunkParams& p, hipStream_t stream) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  const int64_t blocks4 = (p.T + ChunkGeo<4>::Q - 1) / ChunkGeo<4>::Q;
  if (blocks4 * p.heads >= cus || (int64_t)p.T >= (int64_t)ChunkGeo<4>::Q * p.num_reqs) {
    p.nblk = (int)blocks4;
    hipLaunchKernelGGL((chunk_mfma<kWin, 4>), dim3((unsigned)p.nblk * (unsigned)p.heads), dim3(64 * 4), 0, stream, p);
  } else {
    p.nblk = (p.T + ChunkGeo<1>::Q - 1) / ChunkGeo<1>::Q;
    hipLaunchKernelGGL((chunk_mfma<kWin, 1>), dim3((unsigned)p.nblk * (unsigned)p.heads), dim3(64), 0, stream, p);
  }
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
  HLA_REQUIRE((reinterpret_cast<uintptr_t>(out) & 7u) == 0 && o_st % 4 == 0 && o_sh % 4 == 0, HLA_S6_EINVAL,
              "chunk_attention: output rows must be 8-byte aligned");
  ChunkParams p = {};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.q_st = q_st;
  p.q_sh = q_sh;
  p.k_st = k_st;
  p.k_sh = k_sh;
  p.v_st = v_st;
  p.v_sh = v_sh;
  p.qsl = query_start_loc;
  p.num_reqs = num_reqs;
  p.T = num_tokens;
  p.scale_log2 = scale * kLog2e;
  p.out = static_cast<uint16_t*>(out);
  p.o_st = o_st;
  p.o_sh = o_sh;
  p.lse = lse;
  p.heads = num_heads;
  launch_chunk<false>(p, as_stream(stream));
  return check_launch("chunk_attention");
}

extern "C" int hla_s6_chunk_window_attention(const void* q, const void* k, const void* v, int32_t num_tokens,
                                             int32_t num_heads, int32_t head_dim, int64_t q_st, int64_t q_sh,
                                             int64_t k_st, int64_t k_sh, int64_t v_st, int64_t v_sh,
                                             const int32_t* query_start_loc, const int32_t* seq_lens, int32_t num_reqs,
                                             const void* k_cache, const void* v_cache, int64_t page_stride,
                                             int64_t row_stride, int64_t head_stride, int32_t block_size,
                                             int64_t num_blocks, const int32_t* block_table, int64_t bt_stride,
                                             int32_t bt_cols, int32_t window, float scale, void* out, int64_t o_st,
                                             int64_t o_sh, float* lse, void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_tokens >= 0 && num_heads > 0, HLA_S6_EINVAL, "chunk_window_attention: bad token/head count");
  HLA_REQUIRE(head_dim == kExactDim, HLA_S6_EUNSUPPORTED,
              "chunk_window_attention: head_dim %d (the kernel is built for 128)", head_dim);
  HLA_REQUIRE(window >= 0 && block_size > 0 && num_blocks >= 1 && bt_cols >= 0, HLA_S6_EINVAL,
              "chunk_window_attention: bad window, block size, cache size or table width");
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(q && k && v && query_start_loc && seq_lens && num_reqs >= 1 && k_cache && v_cache && block_table &&
                  out && lse,
              HLA_S6_EINVAL, "chunk_window_attention: null pointer or no request");
  HLA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) && aligned16(k_cache) &&
                  aligned16(v_cache) && q_st % 8 == 0 && q_sh % 8 == 0 && k_st % 8 == 0 && k_sh % 8 == 0 &&
                  v_st % 8 == 0 && v_sh % 8 == 0 && o_st % 8 == 0 && o_sh % 8 == 0 && page_stride % 8 == 0 &&
                  row_stride % 8 == 0 && head_stride % 8 == 0,
              HLA_S6_EINVAL, "chunk_window_attention: rows must be 16-byte aligned");
  ChunkParams p = {};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.q_st = q_st;
  p.q_sh = q_sh;
  p.k_st = k_st;
  p.k_sh = k_sh;
  p.v_st = v_st;
  p.v_sh = v_sh;
  p.qsl = query_start_loc;
  p.num_reqs = num_reqs;
  p.T = num_tokens;
  p.scale_log2 = scale * kLog2e;
  p.out = static_cast<uint16_t*>(out);
  p.o_st = o_st;
  p.o_sh = o_sh;
  p.lse = lse;
  p.win.k = static_cast<const uint16_t*>(k_cache);
  p.win.v = static_cast<const uint16_t*>(v_cache);
  p.win.paged = true;
  p.win.page_stride = page_stride;
  p.win.row_stride = row_stride;
  p.win.head_stride = head_stride;
  p.win.num_blocks = num_blocks;
  p.win.block_size = block_size;
  p.bt = block_table;
  p.bt_stride = bt_stride;
  p.bt_cols = bt_cols;
  p.seq_lens = seq_lens;
  p.window = window;
  p.heads = num_heads;
  launch_chunk<true>(p, as_stream(stream));
  return check_launch("chunk_window_attention");
}
