// Paged latent-history attention for the S6 MQA cache (16 query heads share one latent row), and the fused
// decode attention of one layer x loop built on it.
//
// history_split: one workgroup per (token, KV split), one wave per 128 latent columns (4 waves for the 512-wide
// main latent, 2 for the 256-wide loop-1 latent). Wave w owns the latent columns [128w, 128w + 128) of the query,
// of K and of V. Keys are walked in tiles of 16 rows (a tile never crosses a
// page since the page size is a multiple of 16):
//   * S^T[16 keys x 16 heads] = K . Q^T on v_mfma_f32_16x16x32_bf16. Each wave contracts its own 128 columns:
//     K rows are loaded coalesced (4 rows x 256 bytes per instruction), staged in wave-private LDS and read back
//     in the MFMA A-operand layout (lane l: key l%16, 8 consecutive latent columns); Q^T is the B operand, held
//     in registers for the whole row. The per-wave partials are summed through LDS (one barrier per tile, two
//     buffers alternating by tile parity).
//   * online softmax in the exp2 domain on the 4 keys x 1 head each lane owns (cross-lane max/sum over the 4
//     lane groups sharing a head);
//   * O^T[16 cols x 16 heads] += V^T . P^T on v_mfma_f32_16x16x16_bf16: P^T comes straight from the softmax
//     registers (the S^T output layout is the B-operand layout), V^T is read from a wave-private LDS copy of the
//     wave's V columns (transposing 16-bit reads).
//   * the K/V loads of the next tile are in flight while a tile is computed.
// With one split the workgroup writes the final bf16 output and lse. With several, each split writes its
// normalized partial and lse to the fp32 workspace and history_combine (one workgroup per token and head)
// reduces them by LSE in a second launch. (Reducing in the last split of each row instead needs agent-scope
// release fences or L2-bypassing partials; both measured slower on MI355X than the extra launch.)
// For the fused decode step the split workgroups of a token also compute its exact decode window (exact.h), the
// heads spread over the splits, so history and window attention run in one launch; decode_epilogue then reduces
// the split partials, applies B_t and merges with the window in a second one.
#include <mutex>

#include "exact.h"

namespace hla {

namespace {

// Split-kernel constants: latent columns per wave; the compiler is held to 3 waves per SIMD, which keeps the
// accumulators out of AGPRs.
constexpr int kWaveCols = 128;
constexpr int kSplitWavesPerEu = 3;

constexpr int kHeads = 16;
constexpr int kTile = 16;
constexpr int kMaxSplits = 1024;

struct WindowPart {  // decode exact window, computed by the extra row of workgroups
  ExactSource src;
  const uint16_t* q;
  int64_t q_st, q_sh;
  const int32_t* bt;
  int64_t bt_stride;
  int bt_cols;
  const int32_t* qsl;
  const int32_t* seq_lens;
  int num_reqs;
  int window;
  bool chunk_start;  // keys [seq_len - Lq - window, p] (prefill chunks) instead of [p - window, p]
  const int64_t* token_requests;  // request of each token (nullable: searched in qsl)
  uint16_t* out;  // [T, 16, 128]
  int64_t o_st, o_sh;
  float* lse;  // [16, T]
};

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
  float* ws_o;      // [T][S][16][R]
  float* ws_lse;    // [T][S][16]
  uint16_t* out;
  int64_t o_st, o_sh;
  float* lse;  // [16][T]
  const int32_t* plan;  // precomputed split plan of the step (split_plan_kernel) or null
  int group;     // tokens per workgroup (history_group when > 1)
  bool shared_rows;  // tokens re-read the same rows (multi-query steps): cached instead of non-temporal loads
  bool has_window;
  bool direct;   // one split writing the final output and lse (else split partials to the workspace)
  bool combine;  // launch history_combine after the split kernel (with more than one split)
  WindowPart win;
  // contiguous-row form (history_mq2 only): with bt == null, token t reads table row t / tok_per_row whose page p
  // is row * bt_cols + p; lse then goes to [rows, 16, tok_per_row]; mask (when set) hides key j of token t where
  // mask[t * mask_st + j] == 0, or with mask_split mask[row * mask_sb + (t - row * tok_per_row) * mask_st + j] == 0
  // for token t of table row `row` (mask_st 0: one mask row shown to every token of the table row)
  int tok_per_row;
  const uint8_t* mask;
  int64_t mask_st, mask_sb;
  bool mask_split;
  bool lse_rows;  // lse of history_split / history_combine in [rows][16][tok_per_row] instead of [16][T]
  bool reverse_groups;  // history_mq5 / history_group: workgroup b takes token group gridDim.x - 1 - b (the K-hop
                        // causal rows put the longest groups last in token order; dispatching them first shortens
                        // the tail)
};

template <int R>
struct Geo {
  static constexpr int WAVES = R >= kWaveCols ? R / kWaveCols : 1;  // one wave per 128 latent columns
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int QW = R / WAVES;      // latent columns per wave
  static constexpr int KI = QW / 32;        // 16-byte K pieces per lane per tile (= MFMA k-steps)
  static constexpr int VC = QW / 32;        // 16-byte V chunks per lane per tile
  static constexpr int NT = QW / 16;        // 16-column O^T tiles per wave
  static constexpr int CPR = QW / 8;        // 16-byte chunks per V row (wave's columns)
  static constexpr int VS = QW + 16;        // LDS row stride of the K copy, in bf16 (16-byte row reads: +8 conflicts)
  static constexpr int VSV = QW + 16;      // of the V copy (conflict-free transposed reads)
  static constexpr int VBUF = kTile * VSV;  // one wave buffer, in bf16
};

// Split plan shared by the split kernel and the kernels that reduce its partials. Every row of the call is cut in
// chunks of `chunk` 16-row tiles; the grid has S slots per row, and
//   chunk = max(ceil(max_tiles / S), ceil(2 * total_tiles / (T * S)))
// keeps every row within its S slots while about T*S/2 slots get work however ragged the rows are (short rows take
// few slots, long rows many, each holding equal work), and it is at least kMinChunk tiles (kMinChunkSmall in steps
// of fewer than kSmallStepTiles tiles over all rows), or the longest row. Slot s of a row holds tiles
// [s*chunk, (s+1)*chunk); slots past ceil(tiles / chunk) are empty.
//
// The floor: an item's time is a chain of dependent tile steps, its partial costs 16 * (R + 1) fp32 writes and as
// many epilogue reads (as many bytes as a 16-row tile of K and V); a step of many tiles streams, where 8-tile items
// keep that overhead small, and a step of few tiles is latency-bound, where 4-tile items shorten the chain more than
// their partials cost (4-tile items were faster at 256 and 504 tiles per step, 8-tile ones at 1016 and more).
constexpr int kMinChunk = 8, kMinChunkSmall = 4;
constexpr int64_t kSmallStepTiles = 768;
__device__ __forceinline__ int row_tiles(int32_t ctx, int64_t cap) {
  return (int)((min((int64_t)ctx, cap) + kTile - 1) / kTile);
}

// Slots of a row that hold work under a plan of `chunk` tiles.
__device__ __forceinline__ int used_slots(int32_t ctx, int64_t cap, int chunk) {
  return (row_tiles(ctx, cap) + chunk - 1) / chunk;
}

// The plan's chunk. Without `fill`, the formula's chunk grows until the step has at most T*S/2 items: the tails of
// ragged rows add up to T more, and the items past T*S/2 (the split counts aim it at two workgroups per CU) would
// give some CUs a third item, on which the whole call waits. With `fill` (the multi-token kernels, launched on a
// grid of one workgroup per (token group, slot) whether the slot has work or not) it is ceil(max_tiles / S)
// instead: the longest row fills all S slots. Must be called by every thread of the block (a multiple of 64
// threads); `red` holds 2 * waves int64.
__device__ int split_chunk(const int32_t* ctx, int T, int64_t cap, int S, int64_t* red, bool fill = false) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, waves = blockDim.x >> 6;
  const bool one = T <= (int)blockDim.x;  // one row per thread: its tiles stay in a register
  const int my_tiles = tid < T ? row_tiles(ctx[tid], cap) : 0;
  int mx = 0;
  int64_t sum = 0;
  for (int i = tid; i < T; i += blockDim.x) {
    const int tiles = one ? my_tiles : row_tiles(ctx[i], cap);
    mx = max(mx, tiles);
    sum += tiles;
  }
  for (int off = 32; off > 0; off >>= 1) {
    mx = max(mx, __shfl_xor(mx, off));
    sum += __shfl_xor(sum, off);
  }
  if (lane == 0) {
    red[2 * wave] = mx;
    red[2 * wave + 1] = sum;
  }
  __syncthreads();
  int64_t m = 0;
  sum = 0;
  for (int w = 0; w < waves; ++w) {
    m = max(m, red[2 * w]);
    sum += red[2 * w + 1];
  }
  const int64_t slots = (int64_t)T * S;
  int c = (int)max((int64_t)1, fill ? (m + S - 1) / S : max((m + S - 1) / S, (2 * sum + slots - 1) / slots));
  if (fill) return c;
  c = max(c, (int)min(m, (int64_t)(sum < kSmallStepTiles ? kMinChunkSmall : kMinChunk)));
  for (const int64_t target = slots / 2; c < m; ++c) {  // c and the sums are uniform over the block
    int64_t items = 0;
    for (int i = tid; i < T; i += blockDim.x) items += ((one ? my_tiles : row_tiles(ctx[i], cap)) + c - 1) / c;
    for (int off = 32; off > 0; off >>= 1) items += __shfl_xor(items, off);
    __syncthreads();  // every thread has read red
    if (lane == 0) red[wave] = items;
    __syncthreads();
    items = 0;
    for (int w = 0; w < waves; ++w) items += red[w];
    if (items <= target) break;
  }
  __syncthreads();  // red may be reused by the caller
  return c;
}

// Workgroups of the split kernel: the plan puts at most T*S/2 + T (row, chunk) items in the list; a multiple of 8
// (one share per XCD).
__host__ __device__ inline unsigned split_workgroups(int T, int S) {
  return S == 1 ? (unsigned)T : ((unsigned)T * ((S + 1) / 2 + 1) + 7u) / 8u * 8u;
}

// Work item b of the step's list of (row, slot) pairs, rows in order, each row contributing its used slots:
// row = -1 past the end of the list. The split kernel gives item b to the workgroup dispatched b-th, so consecutive
// items land on consecutive XCDs (workgroups are dealt to the XCDs round-robin) and every XCD gets the same share
// of the work, however ragged the rows are. Must be called by every thread (a multiple of 64 threads); `wsum` holds
// one int per wave, `res` two ints.
__device__ void find_item(const int32_t* ctx, int T, int64_t cap, int chunk, int b, int* wsum, int* res, int& row,
                          int& slot) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = blockDim.x;
  const int seg = (T + n - 1) / n, r0 = min(T, tid * seg), r1 = min(T, r0 + seg);
  int cnt = 0;
  for (int r = r0; r < r1; ++r) cnt += used_slots(ctx[r], cap, chunk);
  int x = cnt;  // inclusive scan over the wave
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(x, off);
    if (lane >= off) x += v;
  }
  if (lane == 63) wsum[wave] = x;
  if (tid == 0) res[0] = -1;
  __syncthreads();
  int hi = x;
  for (int w = 0; w < wave; ++w) hi += wsum[w];
  int lo = hi - cnt;
  if (b >= lo && b < hi) {  // exactly one thread owns item b
    for (int r = r0; r < r1; ++r) {
      const int u = used_slots(ctx[r], cap, chunk);
      if (b < lo + u) {
        res[0] = r;
        res[1] = b - lo;
        break;
      }
      lo += u;
    }
  }
  __syncthreads();
  row = res[0];
  slot = res[1];
}

// Plan layout (int32): [0] chunk, [1, 1 + T) used slots per row, then the work items' rows [NI] and slots [NI],
// NI = split_workgroups(T, S); rows past the end of the list are -1.
inline int64_t plan_ints(int T, int S) { return 1 + (int64_t)T + 2 * (int64_t)split_workgroups(T, S); }

// Tokens of one request whose chunks the plan lists chunk-major (at most this many, all with the same slot count)
constexpr int kPlanGroup = 16;

// The split plan of a step, computed once by one workgroup and read by every split kernel of the step (every layer
// and loop with the same lengths and slot count) instead of being derived in each workgroup. The N items, rows in
// order, are cut in 8 contiguous shares of q = ceil(N/8); item i goes to workgroup (i % q) * 8 + i / q, i.e. share
// i / q lands on one XCD (workgroups are dealt to the XCDs round-robin), so every XCD gets the same number of
// items and a row's chunks mostly share an XCD (its query is read from HBM once). With qsl (the step's request
// boundaries), the rows of a request of 2 .. kPlanGroup tokens that all use the same number of slots (a short
// prefill chunk: they read the same latent rows) list their items chunk-major within the request's range: the
// tokens' copies of one chunk are consecutive items, land on one XCD at about the same time and read the chunk's
// rows from HBM once, the other tokens' reads hitting the L2.
// Plans of one step for up to kMaxPlans slot counts (the latent widths' counts), one workgroup each: one launch.
constexpr int kMaxPlans = 4;
struct PlanSet {
  int S[kMaxPlans];
  int32_t* plan[kMaxPlans];
};

__global__ __launch_bounds__(256) void split_plan_kernel(const int32_t* ctx, int T, int64_t cap, PlanSet set,
                                                         const int32_t* qsl, int R) {
  const int S = set.S[blockIdx.x];
  int32_t* plan = set.plan[blockIdx.x];
  __shared__ int64_t red[8];
  __shared__ int wsum[4];
  __shared__ int carry_s;
  __shared__ int xs[256];       // inclusive prefix of the used slots over the rows of a block of 256
  __shared__ int grp[256][3];   // first item of the row's group, rows in the group, row's position in it
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int chunk = split_chunk(ctx, T, cap, S, red);
  const int ni = (int)split_workgroups(T, S);
  int32_t* used = plan + 1;
  int32_t* rows = plan + 1 + T;
  int32_t* slots = rows + ni;
  if (tid == 0) {
    plan[0] = chunk;
    carry_s = 0;
  }
  for (int i = tid; i < ni; i += 256) rows[i] = -1;
  int total = 0;  // items of the step
  const bool one = T <= 256;  // one row per thread: its slot count stays in a register for the list below
  int my_used = 0;
  for (int r = tid; r < T; r += 256) {
    const int u = used_slots(ctx[r], cap, chunk);
    used[r] = u;
    my_used = u;
    total += u;
  }
  for (int off = 32; off > 0; off >>= 1) total += __shfl_xor(total, off);
  if (lane == 0) wsum[wave] = total;
  __syncthreads();
  total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
  const int q = (total + 7) / 8;
  __syncthreads();
  for (int r0 = 0; r0 < T; r0 += 256) {  // rows in blocks of 256: exclusive prefix of the used slots
    const int r = r0 + tid;
    const int u = r < T ? (one ? my_used : used[r]) : 0;
    int x = u;
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(x, off);
      if (lane >= off) x += v;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int local = x;  // inclusive prefix within the block
    for (int w = 0; w < wave; ++w) local += wsum[w];
    const int first = carry_s + local - u;
    // position k of the row in its request's chunk-major group of m rows (k = 0, m = 1: row-major)
    int k = 0, m = 1;
    if (r < T && qsl && r < qsl[R]) {
      const int req = request_of(qsl, R, r), g0 = qsl[req], gm = qsl[req + 1] - g0;
      bool same = gm > 1 && gm <= kPlanGroup;
      for (int e = 0; same && e < gm; ++e) same = used[g0 + e] == u;
      if (same) {
        k = r - g0;
        m = gm;
      }
    }
    xs[tid] = local;
    grp[tid][0] = first - k * u;  // the group's first item (its rows' ranges are contiguous)
    grp[tid][1] = m;
    grp[tid][2] = k;
    __syncthreads();
    // the block's (row, chunk) pairs, spread over the threads: pair p belongs to the first row whose inclusive
    // prefix exceeds p
    const int pairs = xs[255];
    for (int p = tid; p < pairs; p += 256) {
      int lo = 0, hi = 255;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (xs[mid] > p) hi = mid;
        else lo = mid + 1;
      }
      const int c = p - (lo ? xs[lo - 1] : 0);
      const int i = grp[lo][0] + c * grp[lo][1] + grp[lo][2], b = (i % q) * 8 + i / q;
      rows[b] = r0 + lo;
      slots[b] = c;
    }
    __syncthreads();
    if (tid == 255) carry_s += local;
    __syncthreads();
  }
}

template <int R>
struct TileRegs {
  u32x4 k[Geo<R>::KI];
  u32x4 v[Geo<R>::VC];
  uint32_t mk;  // contiguous rows with a key mask: mask bytes of keys 4g .. 4g+3 of the tile (lane group g)
};

// Where history_split's token t finds its rows: a block-table row (paged caches), or the contiguous rows
// [t / tok_per_row] (rows at page_stride, keys at row_stride) with an optional byte mask per (token, key).
struct RowSource {
  const int32_t* btr;    // paged: the token's block-table row
  int64_t base;          // contiguous: element offset of the token's first row
  const uint8_t* mrow;   // contiguous: the token's mask row, or null (every key visible)
};

// K/V row loads: non-temporal when every row is read once (decode), cached when several tokens read the same rows
// (multi-query steps), so that their re-reads hit the L2.
template <bool NT>
__device__ __forceinline__ u32x4 ld_stream(const uint16_t* p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else return ld16(p);
}

template <int R, bool NT, bool kRows = false>
__device__ __forceinline__ void load_tile(const HistoryParams& a, const RowSource& src, int n, int j, int col0,
                                          int lane, TileRegs<R>& r) {
  using G = Geo<R>;
  const int key0 = j * kTile;
  int64_t base;
  if constexpr (kRows) {
    base = src.base + (int64_t)key0 * a.row_stride + col0;
    // mask bytes of keys kb .. kb+3 (one 4-byte load when they are all below the bound and the row is 4-byte
    // aligned; keys at or past the bound are hidden by the bound itself and their bytes are not read)
    const int kb = key0 + 4 * (lane >> 4);
    uint32_t mk = 0xffffffffu;
    if (src.mrow) {
      if (kb + 4 <= n && (reinterpret_cast<uintptr_t>(src.mrow) & 3u) == 0) {
        mk = *reinterpret_cast<const uint32_t*>(src.mrow + kb);
      } else {
        mk = 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (kb + e < n) mk |= (uint32_t)src.mrow[kb + e] << (8 * e);
      }
    }
    r.mk = mk;
  } else {
    const int64_t page = min(max((int64_t)src.btr[key0 / a.block_size], (int64_t)0), a.num_blocks - 1);
    base = page * a.page_stride + (int64_t)(key0 % a.block_size) * a.row_stride + col0;
  }
#pragma unroll
  for (int it = 0; it < G::KI; ++it) {  // same coalesced chunk layout as V: 4 rows x 256 bytes per instruction
    const int c = it * 64 + lane;
    const int key = c / G::CPR;
    r.k[it] = (key0 + key < n) ? ld_stream<NT>(a.k + base + (int64_t)key * a.row_stride + (c % G::CPR) * 8)
                               : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int it = 0; it < G::VC; ++it) {
    const int c = it * 64 + lane;
    const int key = c / G::CPR;
    const int cc = (c % G::CPR) * 8;
    r.v[it] = (key0 + key < n) ? ld_stream<NT>(a.v + base + (int64_t)key * a.row_stride + cc) : u32x4{0u, 0u, 0u, 0u};
  }
}

// Stage A: K and V -> wave-private LDS, the wave's partial of S^T. Consumes the tile registers.
template <int R>
__device__ __forceinline__ floatx4 stage_a(const TileRegs<R>& r, const u32x4 (&qreg)[Geo<R>::KI], uint16_t* vs,
                                           uint16_t* ks, int lane) {
  using G = Geo<R>;
#pragma unroll
  for (int it = 0; it < G::VC; ++it) {
    const int c = it * 64 + lane;
    st16(vs + (c / G::CPR) * G::VSV + (c % G::CPR) * 8, r.v[it]);
  }
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int it = 0; it < G::KI; ++it) {
    const int c = it * 64 + lane;
    st16(ks + (c / G::CPR) * G::VS + (c % G::CPR) * 8, r.k[it]);
  }
  const int hq = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < G::KI; ++i)
    acc = mfma16x16x32(*reinterpret_cast<const u32x4*>(ks + hq * G::VS + 32 * i + 8 * g), qreg[i], acc);
  return acc;
}

// A operand of O^T += V^T P^T for output columns [16nt, 16nt + 16) of the wave's V copy: lane (g, hq) holds
// V[4g + e][16nt + hq], e = 0..3. ds_read_b64_tr_b16 transposes within each 16-lane group: lane j of the group
// reads row 4g + j/4, columns 16nt + 4(j%4) .. +3, and lane i receives element i%4 of lanes 4e + i/4.
template <int R>
__device__ __forceinline__ short4v vt_operand(const uint16_t* vs, int nt, int g, int hq) {
  using G = Geo<R>;
  const uint16_t* p = vs + (4 * g + (hq >> 2)) * G::VSV + 16 * nt + 4 * (hq & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)p);
}

// Stage B: exchange S partials, online softmax, O^T += V^T P^T. With kMask, byte r of mk hides key 4g + r of the
// tile when zero.
template <int R, bool kMask = false>
__device__ __forceinline__ void stage_b(floatx4 sacc, floatx4* sx, const uint16_t* vs, int key0, int n, float scale_log2,
                                        int wave, int lane, floatx4 (&oacc)[Geo<R>::NT], float& m, float& l,
                                        uint32_t mk = 0xffffffffu) {
  using G = Geo<R>;
  sx[wave * 64 + lane] = sacc;
  __syncthreads();
  floatx4 s = sx[lane];
#pragma unroll
  for (int w = 1; w < G::WAVES; ++w) s += sx[w * 64 + lane];
  const int hq = lane & 15, g = lane >> 4;
  const int kb = key0 + 4 * g;
  float sc[4];
  if (kMask) {
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = (kb + r < n && ((mk >> (8 * r)) & 255u) != 0) ? s[r] * scale_log2 : -INFINITY;
  } else if (key0 + kTile <= n) {  // wave-uniform: every key of the tile is history
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = s[r] * scale_log2;
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = (kb + r < n) ? s[r] * scale_log2 : -INFINITY;
  }
  // (scores are finite or -inf: rows past the history are masked before any NaN they hold is used)
  const float mx = wave_max16x4_nn(max_nn(max_nn(sc[0], sc[1]), max_nn(sc[2], sc[3])));
  // the running maximum is raised lazily, only when a tile exceeds it by more than 2^8 (the exponentials stay
  // below 2^8), which skips the rescale of the accumulators on most tiles
  const bool raise = mx > m + 8.f;  // false while the row has no key yet (mx = -inf)
  if (__any(raise)) {
    const float m_new = raise ? mx : m;
    const float alpha = raise ? fast_exp2(m - m_new) : 1.f;  // 0 on the first raise (m = -inf)
    l *= alpha;
    m = m_new;
#pragma unroll
    for (int nt = 0; nt < G::NT; ++nt) oacc[nt] = oacc[nt] * alpha;
  }
  const float m_use = m == -INFINITY ? 0.f : m;
  float p[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) p[r] = fast_exp2(sc[r] - m_use);
  l += (p[0] + p[1]) + (p[2] + p[3]);  // this lane's share of the row sum (the 4 lanes are summed at the end)
  const uint32_t p01 = pack2_hw(p[0], p[1]), p23 = pack2_hw(p[2], p[3]);
  const short4v pb = {(short)(p01 & 0xffffu), (short)(p01 >> 16), (short)(p23 & 0xffffu), (short)(p23 >> 16)};
#pragma unroll
  for (int nt = 0; nt < G::NT; ++nt) {
    const short4v va = vt_operand<R>(vs, nt, g, hq);
    oacc[nt] = mfma16x16x16(va, pb, oacc[nt]);
  }
}

// The decode exact windows of the step, one (token, head) row per wave job: wave v of nv computes rows v, v + nv, ...
// of the 16*T. The split kernel appends window_workgroups() workgroups for them after its history workgroups, so
// the window runs beside the history instead of ahead of it on the first workgroups. A job is a chain of dependent
// loads (request bounds, page table, rows) of several microseconds: a wave takes four with 64 tokens or more
// (hidden behind a long history), one in smaller steps, whose history is short.
__host__ __device__ inline int window_jobs_per_wave(int T) { return T >= 64 ? 4 : 1; }

__host__ __device__ inline unsigned window_workgroups(int T, int waves) {
  const int per = window_jobs_per_wave(T) * waves;
  return (unsigned)((kHeads * T + per - 1) / per);
}

__device__ void window_jobs(const WindowPart& w, int T, float scale_log2, int v, int nv, int lane) {
  for (int j = v; j < kHeads * T; j += nv) {
    const int t = j / kHeads, h = j % kHeads;
    int req, lo, hi;
    decode_window_range(w.qsl, w.seq_lens, w.num_reqs, t, w.window, req, lo, hi, w.chunk_start, w.token_requests);
    ExactSource src = w.src;
    hi = (int)min((int64_t)hi, (int64_t)w.bt_cols * src.block_size);
    src.table_row = w.bt + (int64_t)req * w.bt_stride;
    exact_row(src, w.q + (int64_t)t * w.q_st + (int64_t)h * w.q_sh, scale_log2, lo, hi, h, lane,
              w.out + (int64_t)t * w.o_st + (int64_t)h * w.o_sh, w.lse + (int64_t)h * T + t);
  }
}

// mask bytes of token t whose table row is `row` (contiguous-row forms)
__device__ __forceinline__ const uint8_t* mask_row(const HistoryParams& a, int64_t row, int t) {
  return a.mask + (a.mask_split ? row * a.mask_sb + ((int64_t)t - row * a.tok_per_row) * a.mask_st
                                : (int64_t)t * a.mask_st);
}

// lse index of (token t, head h): [16][T], or [rows][16][tok_per_row] with lse_rows (contiguous rows)
__device__ __forceinline__ int64_t lse_index(const HistoryParams& a, int t, int h) {
  if (!a.lse_rows) return (int64_t)h * a.T + t;
  return ((int64_t)(t / a.tok_per_row) * kHeads + h) * a.tok_per_row + t % a.tok_per_row;
}

// kRows: contiguous rows (bt == null; token t reads rows [t / tok_per_row]) with an optional key mask, whose
// partials may then see no key at all (a zero output and lse = -inf)
template <int R, bool NT, bool kRows = false>
__global__ __launch_bounds__(Geo<R>::THREADS)
__attribute__((amdgpu_waves_per_eu(kSplitWavesPerEu, kSplitWavesPerEu)))
void history_split(HistoryParams a) {
  using G = Geo<R>;
  constexpr int DEPTH = 1, NVB = 1;  // tiles in flight per wave, V copies in LDS
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[G::WAVES][NVB][G::VBUF];
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[G::WAVES][G::VBUF];
  __shared__ floatx4 s_lds[2][G::WAVES * 64];
  __shared__ int64_t red_lds[2 * G::WAVES];
  __shared__ int item_lds[G::WAVES + 2];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int S = a.num_splits;
  const int hq = lane & 15, g = lane >> 4;
  const int64_t cap = (int64_t)a.bt_cols * a.block_size;  // keys the block table can address
  const int b = blockIdx.x;                                 // dispatch order
  const int nh = (int)split_workgroups(a.T, S);  // history workgroups; the ones after them take window jobs
  if (b >= nh) {  // a window workgroup of the fused decode step (uniform over the workgroup)
    window_jobs(a.win, a.T, a.scale_log2, (b - nh) * G::WAVES + wave, (gridDim.x - nh) * G::WAVES, lane);
    return;
  }

  // Split plan: every row is cut in chunks of `chunk` tiles (the same for every row of the step); workgroup b takes
  // the b-th (row, chunk) pair of the step, so the work is balanced over the workgroups and the XCDs.
  int t = b, s = 0, chunk = 0;
  if (S > 1 && a.plan) {
    const int ni = (int)split_workgroups(a.T, S);
    chunk = a.plan[0];
    t = a.plan[1 + a.T + b];
    s = a.plan[1 + a.T + ni + b];
  } else if (S > 1) {
    chunk = split_chunk(a.ctx, a.T, cap, S, red_lds);
    find_item(a.ctx, a.T, cap, chunk, b, item_lds, item_lds + G::WAVES, t, s);
  }
  if (S > 1 && b < a.T) {  // slots of row b past its work: an empty partial for stage 2 (one contiguous range of
                           // lse, written by the whole workgroup: hundreds of slots when the plan leaves most empty)
    const int used = a.plan ? a.plan[1 + b] : used_slots(a.ctx[b], cap, chunk);
    float* l0 = a.ws_lse + ((int64_t)b * S + used) * kHeads;
    for (int i = tid; i < (S - used) * kHeads; i += G::THREADS) l0[i] = -INFINITY;
  }
  if (t < 0) return;  // past the end of the work list (uniform over the workgroup)
  const int n = (int)min((int64_t)a.ctx[t], cap);
  const int tiles = (n + kTile - 1) / kTile;
  if (S == 1) chunk = tiles;
  const int j_begin = s * chunk;
  const int j_end = min(tiles, j_begin + chunk);
  const int col0 = wave * G::QW;
  const int64_t part_row = ((int64_t)t * S + s) * kHeads + hq;

  if (j_begin >= j_end) {  // nothing to read in this split (uniform over the workgroup)
    if (a.direct) {
      uint16_t* op = a.out + (int64_t)t * a.o_st + (int64_t)hq * a.o_sh + col0 + 4 * g;
#pragma unroll
      for (int nt = 0; nt < G::NT; ++nt) *reinterpret_cast<uint2*>(op + 16 * nt) = uint2{0u, 0u};
      if (wave == 0 && g == 0) a.lse[kRows ? lse_index(a, t, hq) : (int64_t)hq * a.T + t] = -INFINITY;
      return;
    }
    if (wave == 0 && g == 0) a.ws_lse[part_row] = -INFINITY;
  } else {
    RowSource src{};
    if constexpr (kRows) {
      const int64_t row = t / a.tok_per_row;
      src.base = row * a.page_stride;
      src.mrow = a.mask ? mask_row(a, row, t) : nullptr;
    } else {
      src.btr = a.bt + (a.bt_rows ? a.bt_rows[t] : (int64_t)t) * a.bt_stride;
    }
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

    // DEPTH register sets: tile j + u lives in regs[u] (compile-time index), refilled with tile j + u + DEPTH as
    // soon as stage A has consumed it. The score exchange alternates between two LDS buffers by tile parity; a
    // wave-private V copy may be reused by the next tile because the wave's own LDS accesses stay in order.
    TileRegs<R> regs[DEPTH];
#pragma unroll
    for (int u = 0; u < DEPTH; ++u)
      if (j_begin + u < j_end) load_tile<R, NT, kRows>(a, src, n, j_begin + u, col0, lane, regs[u]);
    for (int j = j_begin; j < j_end; j += DEPTH) {
#pragma unroll
      for (int u = 0; u < DEPTH; ++u) {
        const int jt = j + u;
        if (jt < j_end) {
          uint16_t* vs = v_lds[wave][jt % NVB];
          floatx4 sa = stage_a<R>(regs[u], qreg, vs, k_lds[wave], lane);
          const uint32_t mk = regs[u].mk;
          if (jt + DEPTH < j_end) load_tile<R, NT, kRows>(a, src, n, jt + DEPTH, col0, lane, regs[u]);
          stage_b<R, kRows>(sa, s_lds[jt & 1], vs, jt * kTile, n, a.scale_log2, wave, lane, oacc, m, l, mk);
        }
      }
    }

    l = wave_sum16x4(l);
    // (with a key mask a split may see no key: l = 0 gives a zero partial with lse = -inf)
    const float inv = kRows ? (l > 0.f ? 1.0f / l : 0.f) : 1.0f / l;
    const float lse = kRows && !(l > 0.f) ? -INFINITY : (m + log2f(l)) * kLn2;
    if (a.direct) {
      uint16_t* op = a.out + (int64_t)t * a.o_st + (int64_t)hq * a.o_sh + col0 + 4 * g;
#pragma unroll
      for (int nt = 0; nt < G::NT; ++nt) {
        const floatx4 o = oacc[nt] * inv;
        *reinterpret_cast<uint2*>(op + 16 * nt) = uint2{pack2(o[0], o[1]), pack2(o[2], o[3])};
      }
      if (wave == 0 && g == 0) a.lse[kRows ? lse_index(a, t, hq) : (int64_t)hq * a.T + t] = lse;
      return;
    }
    float* wp = a.ws_o + part_row * R + col0 + 4 * g;
#pragma unroll
    for (int nt = 0; nt < G::NT; ++nt) *reinterpret_cast<floatx4*>(wp + 16 * nt) = oacc[nt] * inv;
    if (wave == 0 && g == 0) a.ws_lse[part_row] = lse;
  }
}

// ---- multi-query history ------------------------------------------------------------------------------
// history_group: the split kernel for steps with several query rows per request (chunked prefill). One
// workgroup serves NQ consecutive tokens; the tokens that share a block-table row read each K/V tile once.
// Stage A: K and V -> wave-private LDS, the wave's partial of S^T for each of the NQ tokens (the K operand is read
// from LDS once per k-step and reused by every token). Consumes the tile registers.
template <int R, int NQ>
__device__ __forceinline__ void group_stage_a(const TileRegs<R>& r, const u32x4 (&qreg)[NQ][Geo<R>::KI], uint16_t* vs,
                                        uint16_t* ks, int lane, int count, floatx4 (&sacc)[NQ]) {
  using G = Geo<R>;
#pragma unroll
  for (int it = 0; it < G::KI; ++it) {
    const int c = it * 64 + lane;
    st16(vs + (c / G::CPR) * G::VSV + (c % G::CPR) * 8, r.v[it]);
    st16(ks + (c / G::CPR) * G::VS + (c % G::CPR) * 8, r.k[it]);
  }
#pragma unroll
  for (int u = 0; u < NQ; ++u) sacc[u] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int hq = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < G::KI; ++i) {
    const u32x4 kop = *reinterpret_cast<const u32x4*>(ks + hq * G::VS + 32 * i + 8 * g);
#pragma unroll
    for (int u = 0; u < NQ; ++u)
      if (NQ == 1 || u < count) sacc[u] = mfma16x16x32(kop, qreg[u][i], sacc[u]);
  }
}

// Stage B: exchange the S partials, online softmax per token, O^T += V^T P^T (the V^T operand is read once and
// reused by every token). Keys >= n[u] are masked for token u, and with kMask the keys whose byte r of mk[u] is 0
// (keys 4g + r of the tile).
template <int R, int NQ, bool kMask = false>
__device__ __forceinline__ void group_stage_b(const floatx4 (&sacc)[NQ], floatx4* sx, const uint16_t* vs, int key0,
                                        const int (&n)[NQ], int count, float scale_log2, int wave, int lane,
                                        floatx4 (&oacc)[NQ][Geo<R>::NT], float (&m)[NQ], float (&l)[NQ],
                                        const uint32_t (&mk)[NQ]) {
  using G = Geo<R>;
#pragma unroll
  for (int u = 0; u < NQ; ++u) sx[(u * G::WAVES + wave) * 64 + lane] = sacc[u];
  __syncthreads();
  const int hq = lane & 15, g = lane >> 4;
  const int kb = key0 + 4 * g;
    // Several tokens: the running maximum m is only raised (and O rescaled) when a tile's maximum exceeds it by
    // more than kLazy in the exp2 domain, so p <= 2^kLazy and most tiles accumulate into O without a rescale.
    constexpr float kLazy = 8.f;
    short4v pb[NQ];
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      if (u >= count) continue;
      floatx4 s = sx[u * G::WAVES * 64 + lane];
#pragma unroll
      for (int w = 1; w < G::WAVES; ++w) s += sx[(u * G::WAVES + w) * 64 + lane];
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sc[r] = (kb + r < n[u] && (!kMask || ((mk[u] >> (8 * r)) & 255u) != 0)) ? s[r] * scale_log2 : -INFINITY;
      float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      mx = wave_max16x4(mx);
      const bool raise = mx > m[u] + kLazy;  // per head (lane column); false while the token has no key yet
      if (__any(raise)) {
        const float m_new = raise ? mx : m[u];
        const float alpha = raise ? fast_exp2(m[u] - m_new) : 1.f;  // 0 on the first raise (m = -inf)
        l[u] *= alpha;
#pragma unroll
        for (int nt = 0; nt < G::NT; ++nt) oacc[u][nt] = oacc[u][nt] * alpha;
        m[u] = m_new;
      }
      const float m_use = m[u] == -INFINITY ? 0.f : m[u];
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = fast_exp2(sc[r] - m_use);
      l[u] += wave_sum16x4((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
      for (int r = 0; r < 4; ++r) pb[u][r] = (short)f2bf(p[r]);
    }
#pragma unroll
    for (int nt = 0; nt < G::NT; ++nt) {
      const short4v va = vt_operand<R>(vs, nt, g, hq);
#pragma unroll
      for (int u = 0; u < NQ; ++u)
        if (u < count) oacc[u][nt] = mfma16x16x16(va, pb[u], oacc[u][nt]);
    }
}

__device__ __forceinline__ int64_t table_row(const HistoryParams& a, int t) {
  return a.bt_rows ? a.bt_rows[t] : a.tok_per_row > 0 ? (int64_t)(t / a.tok_per_row) : (int64_t)t;
}

// Writes token t's result of split s: the normalized output and lse (one split) or the split partial.
template <int R>
__device__ __forceinline__ void store_split(const HistoryParams& a, int t, int s, int col0, int wave, int lane,
                                            const floatx4 (&oacc)[Geo<R>::NT], float m, float l) {
  using G = Geo<R>;
  const int hq = lane & 15, g = lane >> 4;
  const bool any = l > 0.f;
  const float inv = any ? 1.0f / l : 0.f;
  const float lse = any ? (m + log2f(l)) * kLn2 : -INFINITY;
  if (a.direct) {
    uint16_t* op = a.out + (int64_t)t * a.o_st + (int64_t)hq * a.o_sh + col0 + 4 * g;
#pragma unroll
    for (int nt = 0; nt < G::NT; ++nt) {
      const floatx4 o = oacc[nt] * inv;
      *reinterpret_cast<uint2*>(op + 16 * nt) = uint2{pack2(o[0], o[1]), pack2(o[2], o[3])};
    }
    if (wave == 0 && g == 0) a.lse[lse_index(a, t, hq)] = lse;
    return;
  }
  const int64_t part_row = ((int64_t)t * a.num_splits + s) * kHeads + hq;
  float* wp = a.ws_o + part_row * R + col0 + 4 * g;
#pragma unroll
  for (int nt = 0; nt < G::NT; ++nt) *reinterpret_cast<floatx4*>(wp + 16 * nt) = oacc[nt] * inv;
  if (wave == 0 && g == 0) a.ws_lse[part_row] = lse;
}

// Mask bytes of keys kb .. kb+3 (kb = key0 + 4g) of the pass's tokens tp + u (u < count) of table row `row`: bytes
// at or past a token's bound n[u] are not read (the bound hides those keys); 0xffffffff without a mask.
template <int NQ>
__device__ __forceinline__ void load_token_masks(const HistoryParams& a, int64_t row, int tp, int count,
                                                 const int (&n)[NQ], int key0, int lane, uint32_t (&mk)[NQ]) {
  const int kb = key0 + 4 * (lane >> 4);
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    mk[u] = 0xffffffffu;
    if (!a.mask || u >= count) continue;
    const uint8_t* mr = mask_row(a, row, tp + u);
    if (kb + 4 <= n[u] && (reinterpret_cast<uintptr_t>(mr) & 3u) == 0) {
      mk[u] = *reinterpret_cast<const uint32_t*>(mr + kb);
    } else {
      mk[u] = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (kb + e < n[u]) mk[u] |= (uint32_t)mr[kb + e] << (8 * e);
    }
  }
}

// One workgroup per (group of NQ consecutive tokens, KV split). The tokens of a group that share a block-table row
// (one request of a chunked-prefill step) are processed together, every K/V tile read once for all of them; a
// group that spans several rows takes one pass per row. kRows: contiguous rows (bt == null; token t reads rows
// [t / tok_per_row] at page_stride) with an optional byte mask per (token, key).
template <int R, int NQ, bool kRows = false>
__global__ __launch_bounds__(Geo<R>::THREADS) void history_group(HistoryParams a) {
  using G = Geo<R>;
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[G::WAVES][G::VBUF];
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[G::WAVES][G::VBUF];
  __shared__ floatx4 s_lds[2][NQ * G::WAVES * 64];
  __shared__ int64_t red_lds[2 * G::WAVES];

  const int s = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int S = a.num_splits;
  const int hq = lane & 15, g = lane >> 4;
  const int64_t cap = (int64_t)a.bt_cols * a.block_size;  // keys the block table can address
  const int col0 = wave * G::QW;

  // Split partition: a fixed tile chunk for every row of the step, sized from the longest row, so that rows of a
  // ragged batch get split counts proportional to their length and every split has equal work.
  const int chunk = S > 1 ? split_chunk(a.ctx, a.T, cap, S, red_lds, true) : (1 << 30);
  const int grp = a.reverse_groups ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x;
  const int t_begin = grp * NQ, t_end = min(t_begin + NQ, a.T);

  int par = 0;  // score-exchange buffer of the next tile; alternates over every tile of every pass
  for (int tp = t_begin; tp < t_end;) {
    const int64_t row = table_row(a, tp);
    int te = tp + 1;
    while (te < t_end && table_row(a, te) == row) ++te;
    const int count = te - tp;
    int n[NQ];
    int n_max = 0;
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      n[u] = u < count ? (int)min((int64_t)a.ctx[tp + u], cap) : 0;
      n_max = max(n_max, n[u]);
    }
    const int tiles = (n_max + kTile - 1) / kTile;
    const int j_begin = S > 1 ? s * chunk : 0;
    const int j_end = min(tiles, j_begin + (S > 1 ? chunk : tiles));

    floatx4 oacc[NQ][G::NT];
    float m[NQ], l[NQ];
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      m[u] = -INFINITY;
      l[u] = 0.f;
#pragma unroll
      for (int nt = 0; nt < G::NT; ++nt) oacc[u][nt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    if (j_begin < j_end) {  // uniform over the workgroup
      RowSource src{};
      if constexpr (kRows) src.base = row * a.page_stride;  // (the per-token masks are loaded separately)
      else src.btr = a.bt + row * a.bt_stride;
      u32x4 qreg[NQ][G::KI];
#pragma unroll
      for (int u = 0; u < NQ; ++u) {
        const uint16_t* qp = a.q + (int64_t)(tp + min(u, count - 1)) * a.q_st + (int64_t)hq * a.q_sh + col0 + 8 * g;
#pragma unroll
        for (int i = 0; i < G::KI; ++i) qreg[u][i] = ld16(qp + 32 * i);
      }
      // The next tile's registers are loaded as soon as stage A has consumed the current ones. The score exchange
      // alternates between two LDS buffers, so a wave writing the next tile's partials never touches the buffer
      // a slower wave may still be reading (the barrier in between orders them); the wave-private K/V copies may
      // be rewritten by the next tile because a wave's own LDS accesses stay in order.
      TileRegs<R> regs;
      uint32_t mk[NQ], mk_next[NQ];
#pragma unroll
      for (int u = 0; u < NQ; ++u) mk_next[u] = 0xffffffffu;
      load_tile<R, false, kRows>(a, src, n_max, j_begin, col0, lane, regs);
      if (kRows) load_token_masks<NQ>(a, row, tp, count, n, j_begin * kTile, lane, mk_next);
      for (int jt = j_begin; jt < j_end; ++jt) {
        floatx4 sa[NQ];
        group_stage_a<R, NQ>(regs, qreg, v_lds[wave], k_lds[wave], lane, count, sa);
#pragma unroll
        for (int u = 0; u < NQ; ++u) mk[u] = mk_next[u];
        if (jt + 1 < j_end) {
          load_tile<R, false, kRows>(a, src, n_max, jt + 1, col0, lane, regs);
          if (kRows) load_token_masks<NQ>(a, row, tp, count, n, (jt + 1) * kTile, lane, mk_next);
        }
        group_stage_b<R, NQ, kRows>(sa, s_lds[par], v_lds[wave], jt * kTile, n, count, a.scale_log2, wave, lane,
                                    oacc, m, l, mk);
        par ^= 1;
      }
    }
#pragma unroll
    for (int u = 0; u < NQ; ++u)
      if (u < count) store_split<R>(a, tp + u, s, col0, wave, lane, oacc[u], m[u], l[u]);
    tp = te;
  }
}

// ---- multi-query history (chunked prefill) ------------------------------------------------------------------
constexpr int kMqTokens = 4;              // tokens per workgroup of history_mq2
constexpr int kMqKeys = 32;               // keys per tile

// history_mq2: one workgroup per (group of 4 consecutive tokens, KV slot) with 8 waves; wave w owns token w / 2 (its
// 16 heads are the 16 query rows) and latent column half w % 2. Per 32-key tile:
//   * S^T[32 keys x 16 rows] partial over the wave's R/2 columns on v_mfma_f32_16x16x32_bf16: K rows (A operand)
//     from LDS, Q^T (B operand) in registers for the whole pass;
//   * the two halves of a token swap partials through LDS (one barrier); both waves then hold the full scores and
//     run the same online softmax (a row's 32 keys sit in 4 lanes; the running maximum is raised lazily, only when
//     a tile exceeds it by more than 2^8);
//   * O^T[R/2 columns x 16 rows] += V^T P^T: P^T stays in registers (the score layout is the B-operand layout under
//     a fixed permutation of the 32 keys over the MFMA k index, which V^T follows: two ds_read_b64_tr_b16 per
//     operand, keys 4g.. and 16 + 4g..).
// K tiles are double-buffered in LDS, V single-buffered (a second barrier before its refill); each K and V tile is
// requested about one tile ahead of its LDS store, through registers.
constexpr int kMq2Pages = 2048;  // block-table entries of a pass kept in LDS (longer passes read them from memory)

template <int R>
struct Mq2Geo {
  static constexpr int C = R / 2;                 // latent columns per wave
  static constexpr int KS = C / 32;               // 32-column k-steps of S^T
  static constexpr int CB = C / 16;               // 16-column blocks of O^T
  static constexpr int CPR = R / 8;               // 16-byte pieces per K / V row
  static constexpr int TL = kMqKeys * CPR / 512;  // pieces per thread per tile (K and V each)
  static constexpr int RS = R + 16;               // LDS row stride (bf16): rows 8 banks apart, so the K row reads
                                                  // (8 lanes a cycle) and the transposing V reads are conflict-free
  static_assert(TL >= 1 && KS >= 1, "R must be at least 128");
};

template <int R, bool kContig>
__global__ __launch_bounds__(512) void history_mq2(HistoryParams a) {
  using G = Mq2Geo<R>;
  __shared__ __attribute__((aligned(16))) uint16_t ks_lds[2][kMqKeys * G::RS];
  __shared__ __attribute__((aligned(16))) uint16_t vs_lds[kMqKeys * G::RS];
  __shared__ __attribute__((aligned(16))) floatx4 xs[2][8][2][64];  // S^T partials [tile parity][wave][key block]
  __shared__ int32_t pg_lds[kMq2Pages];                              // the pass's pages (block-table entries)
  __shared__ int64_t red_lds[16];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, g = lane >> 4;
  const int u = wave >> 1, half = wave & 1, col0 = half * G::C;
  const int S = a.num_splits, s = blockIdx.y;
  const int64_t cap = (int64_t)a.bt_cols * a.block_size;
  const int chunk = S > 1 ? split_chunk(a.ctx, a.T, cap, S, red_lds, true) : (1 << 30);
  const int t_begin = blockIdx.x * kMqTokens, t_end = min(t_begin + kMqTokens, a.T);
  int par = 0;  // parity of the partial exchange buffer, continued across passes

  for (int tp = t_begin; tp < t_end;) {  // passes: runs of tokens that share a table row
    const int64_t row = table_row(a, tp);
    int te = tp + 1;
    while (te < t_end && table_row(a, te) == row) ++te;
    const int count = te - tp;
    int n_max = 0, n_own = 0;
#pragma unroll
    for (int v = 0; v < kMqTokens; ++v) {
      const int n = v < count ? (int)min((int64_t)a.ctx[tp + v], cap) : 0;
      n_max = max(n_max, n);
      if (v == u) n_own = n;
    }
    const int tiles16 = (n_max + kTile - 1) / kTile;
    const int j0 = S > 1 ? s * chunk : 0;
    const int j1 = S > 1 ? min(tiles16, j0 + chunk) : tiles16;
    const int k0 = j0 * kTile, k1 = min(n_max, j1 * kTile);
    const int own_n = min(k1, n_own);
    float m_own = -INFINITY, l_own = 0.f;
    floatx4 o[G::CB];
#pragma unroll
    for (int cb = 0; cb < G::CB; ++cb) o[cb] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (k0 < k1) {  // uniform over the workgroup
      const int32_t* btr = kContig ? nullptr : a.bt + row * a.bt_stride;
      const int tq = tp + min(u, count - 1);
      const uint8_t* mrow = kContig && a.mask ? mask_row(a, row, tq) : nullptr;
      u32x4 qf[G::KS];
      {
        const uint16_t* qp = a.q + (int64_t)tq * a.q_st + (int64_t)l16 * a.q_sh + col0 + 8 * g;
#pragma unroll
        for (int k = 0; k < G::KS; ++k) qf[k] = ld16(qp + 32 * k);
      }
      // the pass's block-table entries go to LDS once, so no K / V load waits on a dependent table load
      const int p0 = k0 / a.block_size, np = (k1 - 1) / a.block_size - p0 + 1;
      const bool pg_local = np <= kMq2Pages;
      __syncthreads();  // the previous pass's readers of the tiles and pages are done
      auto table_page = [&](int p) -> int64_t {  // clamped entry p of the row (identity pages: contiguous rows)
        return kContig ? row * a.bt_cols + p : min(max((int64_t)btr[p], (int64_t)0), a.num_blocks - 1);
      };
      if (pg_local)
        for (int i = tid; i < np; i += 512) pg_lds[i] = (int32_t)table_page(p0 + i);
      __syncthreads();
      auto page_of = [&](int key) -> int64_t {
        const int p = key / a.block_size;
        return pg_local ? (int64_t)pg_lds[p - p0] : table_page(p);
      };
      u32x4 kr[G::TL], vr[G::TL];
      // piece c = it * 512 + tid of a tile: key kt + c / CPR, 16-byte piece c % CPR. With 16-row pages (tiles start
      // on a page) the page is entry kt / 16 + (c / CPR) / 16 and the row (c / CPR) % 16: fixed offsets per thread.
      const bool page16 = a.block_size == kTile;
      auto load = [&](u32x4(&r)[G::TL], const uint16_t* base, int kt) {
#pragma unroll
        for (int it = 0; it < G::TL; ++it) {
          const int c = it * 512 + tid, kr_ = c / G::CPR;
          const int key = min(kt + kr_, k1 - 1);
          int64_t off;
          if (page16 && pg_local && kt + kMqKeys <= k1)
            off = (int64_t)pg_lds[(kt >> 4) - p0 + (kr_ >> 4)] * a.page_stride + (int64_t)(kr_ & 15) * a.row_stride;
          else
            off = page_of(key) * a.page_stride + (int64_t)(key % a.block_size) * a.row_stride;
          r[it] = ld16(base + off + (c % G::CPR) * 8);
        }
      };
      auto store = [&](uint16_t* tile, const u32x4(&r)[G::TL]) {
#pragma unroll
        for (int it = 0; it < G::TL; ++it) {
          const int c = it * 512 + tid;
          st16(tile + (c / G::CPR) * G::RS + (c % G::CPR) * 8, r[it]);
        }
      };
      load(kr, a.k, k0);
      load(vr, a.v, k0);
      store(ks_lds[0], kr);
      store(vs_lds, vr);
      __syncthreads();
      if (k0 + kMqKeys < k1) {
        load(kr, a.k, k0 + kMqKeys);
        load(vr, a.v, k0 + kMqKeys);
      }
      int buf = 0;
      // tile i: K(i + 1) goes to the other K buffer before the exchange barrier and K(i + 2) is requested right
      // after it; V(i + 1) replaces V(i) after the P V barrier and V(i + 2) is requested then: every load has about
      // one tile of time before it is needed
      for (int kt = k0; kt < k1; kt += kMqKeys) {
        const bool more = kt + kMqKeys < k1, more2 = kt + 2 * kMqKeys < k1;
        {  // S^T partials over this wave's columns
          const uint16_t* kp = ks_lds[buf] + l16 * G::RS + col0 + 8 * g;
          floatx4 sp[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
          for (int k = 0; k < G::KS; ++k) {
            sp[0] = mfma16x16x32(*reinterpret_cast<const u32x4*>(kp + 32 * k), qf[k], sp[0]);
            sp[1] = mfma16x16x32(*reinterpret_cast<const u32x4*>(kp + 16 * G::RS + 32 * k), qf[k], sp[1]);
          }
          xs[par][wave][0][lane] = sp[0];
          xs[par][wave][1][lane] = sp[1];
        }
        if (more) store(ks_lds[buf ^ 1], kr);  // every wave finished reading that buffer before the last barrier
        __syncthreads();
        if (more2) load(kr, a.k, kt + 2 * kMqKeys);
        float p[2][4];
        {  // full scores (own + partner partial), online softmax of row l16 (keys 16kb + 4g + r in this lane)
          const floatx4 mine0 = xs[par][wave][0][lane], mine1 = xs[par][wave][1][lane];
          const floatx4 other0 = xs[par][wave ^ 1][0][lane], other1 = xs[par][wave ^ 1][1][lane];
          float sc[2][4];
          // wave-uniform: no key of the tile is past the row's history and no mask applies
          const bool full = kt + kMqKeys <= own_n && (!kContig || !mrow);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float s0 = (half == 0 ? mine0[r] + other0[r] : other0[r] + mine0[r]) * a.scale_log2;
            const float s1 = (half == 0 ? mine1[r] + other1[r] : other1[r] + mine1[r]) * a.scale_log2;
            const int j0 = kt + 4 * g + r, j1 = kt + 16 + 4 * g + r;
            sc[0][r] = full || (j0 < own_n && (!kContig || !mrow || mrow[j0])) ? s0 : -INFINITY;
            sc[1][r] = full || (j1 < own_n && (!kContig || !mrow || mrow[j1])) ? s1 : -INFINITY;
          }
          float mx = sc[0][0];
#pragma unroll
          for (int r = 0; r < 4; ++r) mx = fmaxf(mx, fmaxf(sc[0][r], sc[1][r]));
          mx = wave_max16x4(mx);
          const bool raise = mx > m_own + 8.f;  // false while the row has no key yet (mx = -inf)
          if (__any(raise)) {
            const float m_new = raise ? mx : m_own;
            const float alpha = raise ? fast_exp2(m_own - m_new) : 1.f;  // 0 on the first raise (m_own = -inf)
            l_own *= alpha;
            m_own = m_new;
#pragma unroll
            for (int cb = 0; cb < G::CB; ++cb) o[cb] *= alpha;
          }
          const float m_use = m_own == -INFINITY ? 0.f : m_own;
          float ps = 0.f;
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              p[kb][r] = fast_exp2(sc[kb][r] - m_use);
              ps += p[kb][r];
            }
          ps = wave_sum16x4(ps);
          l_own += ps;
        }
        {  // O^T += V^T P^T (k slot 8g + e <-> key 4g + e, e < 4; key 16 + 4g + e - 4, e >= 4)
          const u32x4 pb = {pack2(p[0][0], p[0][1]), pack2(p[0][2], p[0][3]), pack2(p[1][0], p[1][1]),
                            pack2(p[1][2], p[1][3])};
          const uint16_t* vp = vs_lds + (4 * g + (l16 >> 2)) * G::RS + col0 + 4 * (l16 & 3);
#pragma unroll
          for (int cb = 0; cb < G::CB; ++cb) {
            const short4v lo =
                __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)(vp + 16 * cb));
            const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) short4v*)(vp + 16 * G::RS + 16 * cb));
            const u32x4 vt = join_tr(lo, hi);
            o[cb] = mfma16x16x32(vt, pb, o[cb]);
          }
        }
        par ^= 1;
        if (more) {
          __syncthreads();  // every wave's P V of this tile is done with the V buffer
          store(vs_lds, vr);
          if (more2) load(vr, a.v, kt + 2 * kMqKeys);
          buf ^= 1;
        }
      }
    }
    if (u < count) {  // lane holds O^T[col 16cb + 4g + r][head l16] of token tp + u
      const int t = tp + u, h = l16;
      const bool any = l_own > 0.f;
      const float inv = any ? 1.0f / l_own : 0.f;
#pragma unroll
      for (int cb = 0; cb < G::CB; ++cb) {
        const int col = col0 + 16 * cb + 4 * g;
        const floatx4 v = o[cb] * inv;
        if (a.direct)
          *reinterpret_cast<uint2*>(a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh + col) =
              uint2{pack2(v[0], v[1]), pack2(v[2], v[3])};
        else
          *reinterpret_cast<floatx4*>(a.ws_o + (((int64_t)t * S + s) * kHeads + h) * R + col) = v;
      }
      if (half == 0 && g == 0) {
        const float lse = any ? (m_own + log2f(l_own)) * kLn2 : -INFINITY;
        if (kContig)
          a.lse[((int64_t)(t / a.tok_per_row) * kHeads + h) * a.tok_per_row + t % a.tok_per_row] = lse;
        else if (a.direct) a.lse[(int64_t)h * a.T + t] = lse;
        else a.ws_lse[((int64_t)t * S + s) * kHeads + h] = lse;
      }
    }
    tp = te;
  }
}

constexpr int kMq4Tokens = 8;           // tokens per workgroup of history_mq5
constexpr int kMq4Keys = 32;            // keys per tile
constexpr bool kKhopReverse = true;     // K-hop forward: token groups dispatched last to first
constexpr int kKhop1024Tokens = 2;      // tokens per workgroup of the 1024-wide K-hop forward (history_group)

// history_mq5: one workgroup per (group of 8 consecutive tokens, KV slot); each wave owns TPW tokens of the pass
// and all R latent columns, so its scores need no exchange with another wave: per 32-key tile it computes S^T for
// its tokens (every K fragment read from LDS feeds their MFMAs), runs an online softmax per query row (a row's 32
// keys sit in 4 lanes; NaN-free max3 chains and permlane swaps for the cross-lane steps; the running maximum is
// raised lazily, only when a tile exceeds it by more than 2^8; each lane keeps its share of the row sum) and adds
// V^T P^T with P^T in registers (the score layout is the B-operand layout under a fixed permutation of the 32 keys
// over the MFMA k index, which the two transposing reads of V^T follow). K and V tiles go global -> LDS by direct
// copies (global_load_lds_dwordx4, 16 bytes per lane, one row per instruction: half a wave for a 512-byte row, the
// whole wave for a 1 KB one; wave w copying rows 32 / NW * w ..) into four buffers (K and V of tiles i and i+1);
// one barrier per tile, after which tile i+2 replaces tile i, so every copy has a tile of time. The copies are
// waited for explicitly (s_waitcnt vmcnt counting the copies issued after the awaited ones) and the loop
// synchronizes with plain s_barrier behind those waits, so a copy still in flight for a later tile is never waited
// for at a barrier.
//   R = 512: 8 waves of 1 token (the registers hold 16 query rows x 512 columns), 139 KB of LDS;
//   R = 256: 74 KB of LDS; 4 waves of 2 tokens when the grid has more workgroups than CUs (two workgroups per CU,
//   whose tiles run out of step), else 8 waves of 1 token (one workgroup per CU at two waves per SIMD instead of
//   one).
constexpr int kMq5Pages = 1024;  // block-table entries of a pass kept in LDS (longer passes read them from memory)

template <int R, int kTpw = 1>
struct Mq5Geo {
  static constexpr int TPW = kTpw;              // tokens per wave
  static constexpr int NW = kMq4Tokens / TPW;   // waves per workgroup
  static constexpr int RPW = kMq4Keys / NW;     // tile rows each wave copies (K and V each)
};

template <int R, int kMode, int kTpw = 1>
__global__ __launch_bounds__((64 * Mq5Geo<R, kTpw>::NW), R == 256 ? 2 : 1) void history_mq5(HistoryParams a) {
  static_assert(R == 256 || R == 512, "rows of 512 B (half a copy instruction) or 1 KB");
  using G = Mq5Geo<R, kTpw>;
  constexpr int TPW = G::TPW, NW = G::NW, RPW = G::RPW;
  constexpr bool kContig = kMode != 0, kMask = kMode == 2;
  constexpr int TOPS = 2 * RPW + (kMask ? 1 : 0);  // copy instructions per wave for a tile (K, V rows, mask)
  constexpr int KS = R / 32, CB = R / 16, RS = R + 16;
  __shared__ __attribute__((aligned(16))) uint16_t kt_lds[2][kMq4Keys * RS];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[2][kMq4Keys * RS];
  __shared__ __attribute__((aligned(16))) uint8_t mk_lds[kMask ? 2 : 1][NW][32 * TPW];  // [parity][wave][token*32+key]
  __shared__ int32_t pg_lds[kMq5Pages];
  __shared__ int64_t red_lds[8];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int S = a.num_splits, s = blockIdx.y;
  const int64_t cap = (int64_t)a.bt_cols * a.block_size;
  const int chunk = S > 1 ? split_chunk(a.ctx, a.T, cap, S, red_lds, true) : (1 << 30);
  const int grp = a.reverse_groups ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x;
  const int t_begin = grp * kMq4Tokens, t_end = min(t_begin + kMq4Tokens, a.T);

  for (int tp = t_begin; tp < t_end;) {  // passes: runs of tokens that share a table row
    const int64_t row = table_row(a, tp);
    int te = tp + 1;
    while (te < t_end && table_row(a, te) == row) ++te;
    const int count = te - tp;
    int n_max = 0, n_tok[TPW];
#pragma unroll
    for (int x = 0; x < TPW; ++x) n_tok[x] = 0;
#pragma unroll
    for (int v = 0; v < kMq4Tokens; ++v) {
      const int n = v < count ? (int)min((int64_t)a.ctx[tp + v], cap) : 0;
      n_max = max(n_max, n);
#pragma unroll
      for (int x = 0; x < TPW; ++x)
        if (v == TPW * wave + x) n_tok[x] = n;
    }
    const int tiles16 = (n_max + kTile - 1) / kTile;
    const int j0 = S > 1 ? s * chunk : 0;
    const int j1 = S > 1 ? min(tiles16, j0 + chunk) : tiles16;
    const int k0 = j0 * kTile, k1 = min(n_max, j1 * kTile);
    int own_n[TPW];
    float m_own[TPW], l_own[TPW];
    floatx4 o[TPW][CB];
#pragma unroll
    for (int x = 0; x < TPW; ++x) {
      own_n[x] = min(k1, n_tok[x]);
      m_own[x] = -INFINITY;
      l_own[x] = 0.f;
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) o[x][cb] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    if (k0 < k1) {  // uniform over the workgroup
      const int32_t* btr = kContig ? nullptr : a.bt + row * a.bt_stride;
      u32x4 qf[TPW][KS];
#pragma unroll
      for (int x = 0; x < TPW; ++x) {
        const int tq = tp + min(TPW * wave + x, count - 1);
        const uint16_t* qp = a.q + (int64_t)tq * a.q_st + (int64_t)l16 * a.q_sh + 8 * g;
#pragma unroll
        for (int k = 0; k < KS; ++k) qf[x][k] = ld16(qp + 32 * k);
      }
      const int p0 = k0 / a.block_size, np = (k1 - 1) / a.block_size - p0 + 1;
      const bool pg_local = np <= kMq5Pages;
      __syncthreads();  // the previous pass's readers of the tiles and pages are done
      auto table_page = [&](int p) -> int64_t {  // clamped entry p of the row (identity pages: contiguous rows)
        return kContig ? row * a.bt_cols + p : min(max((int64_t)btr[p], (int64_t)0), a.num_blocks - 1);
      };
      if (pg_local)
        for (int i = tid; i < np; i += 64 * NW) pg_lds[i] = (int32_t)table_page(p0 + i);
      __syncthreads();
      // the query loads are complete before the first copy: the compiler does not see the copies, so no wait it
      // places for an earlier load may end up counting them
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
      const bool page16 = a.block_size == kTile;
      const uint32_t voff = 16u * lane;
      // rows RPW * wave .. of the tile at key kt into buffer buf (keys past the slot's range read its last row)
      auto copy_rows = [&](uint16_t* buf, const uint16_t* base, int kt) {
        const int r0 = RPW * wave;
        if (page16 && pg_local && kt + kMq4Keys <= k1) {  // the RPW rows sit in page kt / 16 + r0 / 16
          const int64_t page = __builtin_amdgcn_readfirstlane(pg_lds[(kt >> 4) - p0 + (r0 >> 4)]);
          const uint16_t* src = base + page * a.page_stride + (int64_t)(r0 & 15) * a.row_stride;
#pragma unroll
          for (int i = 0; i < RPW; ++i)
            if (R == 512 || lane < 32) copy16_to_lds(src + i * a.row_stride, voff, &buf[(r0 + i) * RS]);
        } else {
#pragma unroll
          for (int i = 0; i < RPW; ++i) {
            const int key = min(kt + r0 + i, k1 - 1), p = key / a.block_size;
            const int64_t page = uniform64(pg_local ? (int64_t)pg_lds[p - p0] : table_page(p));
            if (R == 512 || lane < 32)
              copy16_to_lds(base + page * a.page_stride + (int64_t)(key % a.block_size) * a.row_stride, voff,
                            &buf[(r0 + i) * RS]);
          }
        }
      };
      // lane l < 2 TPW copies mask bytes of the wave's token l / 2
      const uint8_t* mk_src = kMask ? mask_row(a, row, tp + min(TPW * wave + (lane >> 1), count - 1)) : nullptr;
      auto copy_tile = [&](int j) {  // tile j (K, V and this wave's mask bytes) into the buffers of parity j & 1
        const int kt = k0 + j * kMq4Keys;
        if (kMask && lane < 2 * TPW) {  // token l / 2, bytes 16 (l % 2) .. (chunks past the row: its end)
          const int c0 = min(kt + 16 * (lane & 1), (int)cap - 16);
          copy16_to_lds_v(mk_src + c0, &mk_lds[j & 1][wave][0]);
        }
        copy_rows(kt_lds[j & 1], a.k, kt);
        copy_rows(vt_lds[j & 1], a.v, kt);
      };
      const int ntiles = (k1 - k0 + kMq4Keys - 1) / kMq4Keys;
      copy_tile(0);
      if (ntiles > 1) {
        copy_tile(1);
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(TOPS, 15));  // tile 0 landed; tile 1 may be in flight
      } else {
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
      }
      plain_barrier();
      for (int i = 0; i < ntiles; ++i) {
        const int kt = k0 + i * kMq4Keys, par = i & 1;
        floatx4 sp[TPW][2];  // S^T of the wave's tokens: keys 16 kb + 4g + r, row l16
        {
          const uint16_t* kp = &kt_lds[par][l16 * RS + 8 * g];
#pragma unroll
          for (int x = 0; x < TPW; ++x) sp[x][0] = sp[x][1] = floatx4{0.f, 0.f, 0.f, 0.f};
          u32x4 ka = *reinterpret_cast<const u32x4*>(kp), kc = *reinterpret_cast<const u32x4*>(kp + 16 * RS);
#pragma unroll
          for (int k = 0; k < KS; ++k) {  // the next k-step's fragments are requested before this one's MFMAs
            const u32x4 ca = ka, cc = kc;
            if (k + 1 < KS) {
              ka = *reinterpret_cast<const u32x4*>(kp + 32 * (k + 1));
              kc = *reinterpret_cast<const u32x4*>(kp + 16 * RS + 32 * (k + 1));
            }
#pragma unroll
            for (int x = 0; x < TPW; ++x) {
              sp[x][0] = mfma16x16x32(ca, qf[x][k], sp[x][0]);
              sp[x][1] = mfma16x16x32(cc, qf[x][k], sp[x][1]);
            }
          }
        }
        auto softmax_tok = [&](int x) -> u32x4 {  // online softmax of row l16 of token x; P^T as the B operand
          const int n = own_n[x];
          float sc[2][4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            sc[0][r] = sp[x][0][r];
            sc[1][r] = sp[x][1][r];
          }
          if (kMask) {  // mask bytes of keys 4g + r and 16 + 4g + r of token x
            const uint8_t* mb = &mk_lds[par][wave][32 * x + 4 * g];
            const uint32_t m0 = *reinterpret_cast<const uint32_t*>(mb), m1 = *reinterpret_cast<const uint32_t*>(mb + 16);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if (kt + 4 * g + r >= n || ((m0 >> (8 * r)) & 255u) == 0) sc[0][r] = -INFINITY;
              if (kt + 16 + 4 * g + r >= n || ((m1 >> (8 * r)) & 255u) == 0) sc[1][r] = -INFINITY;
            }
          } else if (kt + kMq4Keys > n) {  // wave-uniform: the tile runs past the row's history
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if (kt + 4 * g + r >= n) sc[0][r] = -INFINITY;
              if (kt + 16 + 4 * g + r >= n) sc[1][r] = -INFINITY;
            }
          }
          // (scores are finite or -inf: rows past the history are masked before any NaN they hold is used)
          float mx = max3_nn(max3_nn(sc[0][0], sc[0][1], sc[0][2]), max3_nn(sc[0][3], sc[1][0], sc[1][1]),
                             max_nn(sc[1][2], sc[1][3]));
          // the scale is positive, so the maximum of the scaled scores is the scaled maximum (log2 units)
          mx = wave_max16x4_nn(mx) * a.scale_log2;
          const bool raise = mx > m_own[x] + 8.f;  // false while the row has no key yet (mx = -inf)
          if (__any(raise)) {
            const float m_new = raise ? mx : m_own[x];
            const float alpha = raise ? fast_exp2(m_own[x] - m_new) : 1.f;  // 0 on the first raise (m_own = -inf)
            l_own[x] *= alpha;  // this lane's share of the row sum
            m_own[x] = m_new;
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) o[x][cb] *= alpha;
          }
          const float m_use = m_own[x] == -INFINITY ? 0.f : m_own[x];
          float p[2][4], ps = 0.f;
#pragma unroll
          for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              p[kb2][r] = fast_exp2(__builtin_fmaf(sc[kb2][r], a.scale_log2, -m_use));
              ps += p[kb2][r];
            }
          l_own[x] += ps;  // the four lanes of a row are summed once, after the last tile
          return u32x4{pack2_hw(p[0][0], p[0][1]), pack2_hw(p[0][2], p[0][3]), pack2_hw(p[1][0], p[1][1]),
                       pack2_hw(p[1][2], p[1][3])};
        };
        // O^T += V^T P^T (k slot 8g + e <-> key 4g + e, e < 4; key 16 + 4g + e - 4, e >= 4)
        const uint16_t* vp = &vt_lds[par][(4 * g + (l16 >> 2)) * RS + 4 * (l16 & 3)];
        auto vfrag = [&](int cb) {
          const short4v lo =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)(vp + 16 * cb));
          const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) short4v*)(vp + 16 * RS + 16 * cb));
          return join_tr(lo, hi);
        };
        {
          u32x4 pb[TPW];
#pragma unroll
          for (int x = 0; x < TPW; ++x) pb[x] = softmax_tok(x);
          u32x4 vt = vfrag(0);
#pragma unroll
          for (int cb = 0; cb < CB; ++cb) {  // the next fragment is requested before this one's MFMAs; it feeds
            const u32x4 cur = vt;           // every token's MFMA
            if (cb + 1 < CB) vt = vfrag(cb + 1);
#pragma unroll
            for (int x = 0; x < TPW; ++x) o[x][cb] = mfma16x16x32(cur, pb[x], o[x][cb]);
          }
        }
        if (i + 1 < ntiles) {
          // tile i+1 landed (nothing newer is in flight); every wave is done with tile i's buffers
          __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
          plain_barrier();
          if (i + 2 < ntiles) copy_tile(i + 2);  // tile i+2 into tile i's buffers
        }
      }
    }
#pragma unroll
    for (int x = 0; x < TPW; ++x) l_own[x] = wave_sum16x4(l_own[x]);
#pragma unroll
    for (int x = 0; x < TPW; ++x) {
      if (TPW * wave + x >= count) continue;
      const int t = tp + TPW * wave + x, h = l16;  // lane holds O^T[col 16cb + 4g + r][head l16] of token t
      const bool any = l_own[x] > 0.f;
      const float inv = any ? 1.0f / l_own[x] : 0.f;
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int col = 16 * cb + 4 * g;
        const floatx4 v = o[x][cb] * inv;
        if (a.direct)
          *reinterpret_cast<uint2*>(a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh + col) =
              uint2{pack2(v[0], v[1]), pack2(v[2], v[3])};
        else
          *reinterpret_cast<floatx4*>(a.ws_o + (((int64_t)t * S + s) * kHeads + h) * R + col) = v;
      }
      if (g == 0) {
        const float lse = any ? (m_own[x] + log2f(l_own[x])) * kLn2 : -INFINITY;
        if (kContig)
          a.lse[((int64_t)(t / a.tok_per_row) * kHeads + h) * a.tok_per_row + t % a.tok_per_row] = lse;
        else if (a.direct) a.lse[(int64_t)h * a.T + t] = lse;
        else a.ws_lse[((int64_t)t * S + s) * kHeads + h] = lse;
      }
    }
    tp = te;
  }
}

// Split reduction: one workgroup per (token, head) of 4 slot groups x R/4 threads; thread (group q, i) owns output
// columns [4i, 4i+4) of the slots s = q (mod 4), and the 4 groups' sums are added in LDS in a fixed order.
constexpr int kCombineGroups = 4;
template <int R>
constexpr int combine_threads() { return kCombineGroups * (R / 4); }

template <int R>
__global__ __launch_bounds__(combine_threads<R>()) void history_combine(HistoryParams a) {
  constexpr int CT = R / 4, NG = kCombineGroups;
  __shared__ int64_t red[2 * combine_threads<R>() / 64];
  __shared__ float mx_s[NG];
  __shared__ floatx4 acc_s[NG - 1][CT];
  __shared__ float den_s[NG - 1];
  const int t = blockIdx.x, h = blockIdx.y, i = threadIdx.x % CT, q = threadIdx.x / CT;
  const int S_all = a.num_splits;
  // slots past the row's work hold lse = -inf; with the lengths at hand they are not read at all
  int S = S_all;
  if (a.ctx) {
    const int64_t cap = (int64_t)a.bt_cols * a.block_size;
    S = min(S_all, used_slots(a.ctx[t], cap, split_chunk(a.ctx, a.T, cap, S_all, red, a.group > 1)));
  }
  const float* ls = a.ws_lse + (int64_t)t * S_all * kHeads + h;
  float mq = -INFINITY;
  for (int s = q; s < S; s += NG) mq = fmaxf(mq, ls[(int64_t)s * kHeads]);
  if (i == 0) mx_s[q] = mq;
  __syncthreads();
  float mx = mx_s[0];
#pragma unroll
  for (int g = 1; g < NG; ++g) mx = fmaxf(mx, mx_s[g]);
  uint16_t* op = a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh + 4 * i;
  if (mx == -INFINITY) {  // uniform over the workgroup
    if (q == 0) *reinterpret_cast<uint2*>(op) = uint2{0u, 0u};
    if (q == 0 && i == 0) a.lse[lse_index(a, t, h)] = -INFINITY;
    return;
  }
  const float* base = a.ws_o + ((int64_t)t * S_all * kHeads + h) * R + 4 * i;
  // Eight of the group's partial rows in flight. One code path for every slot count (a slot past S or without work
  // adds an exact zero through fma(0, 0, acc)), so the result does not depend on how many empty slots are read.
  float den = 0.f;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = q; s0 < S; s0 += 8 * NG) {
    floatx4 o[8];
    float w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int sl = s0 + u * NG;
      const bool in = sl < S;
      o[u] = in ? *reinterpret_cast<const floatx4*>(base + (int64_t)sl * kHeads * R) : floatx4{0.f, 0.f, 0.f, 0.f};
      const float l_s = in ? ls[(int64_t)sl * kHeads] : -INFINITY;
      w[u] = l_s == -INFINITY ? 0.f : __expf(l_s - mx);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      den += w[u];
      const floatx4 ou = w[u] == 0.f ? floatx4{0.f, 0.f, 0.f, 0.f} : o[u];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(ou[e], w[u], acc[e]);
    }
  }
  if (q > 0) {
    acc_s[q - 1][i] = acc;
    if (i == 0) den_s[q - 1] = den;
  }
  __syncthreads();
  if (q != 0) return;
#pragma unroll
  for (int g = 0; g < NG - 1; ++g) {
    acc += acc_s[g][i];
    den += den_s[g];
  }
  acc = acc * (1.0f / den);
  *reinterpret_cast<uint2*>(op) = uint2{pack2(acc[0], acc[1]), pack2(acc[2], acc[3])};
  if (i == 0) a.lse[lse_index(a, t, h)] = mx + logf(den);
}

// ---- decode epilogue --------------------------------------------------------------------------------------------
// out[t, h, :] = merge(bf16(o_hist[t, h, :] @ B[h]), o_win[t, h, :]) for TB tokens of one head per workgroup of W
// waves (4 tokens and 4 waves, or 1 token and 8 waves for small steps, so that the split reduction spreads over
// enough workgroups and each round of loads covers enough slots):
//   1. o_hist: LSE reduction of the split partials (or the direct bf16 output with one split), rounded to bf16 as the
//      history op's output is, kept in LDS as bf16 pairs;
//   2. the B_t product as a GEMV on bf16 pairs: wave q sums rows [q*R/W, (q+1)*R/W) of B[h]; lane (g, c) =
//      (lane/16, lane%16) reads rows k = 8*step + 2g and k + 1, output columns [8c, 8c+8) (16-byte loads: a wave
//      instruction covers 4 whole B rows), pairs the two rows' values of each column (v_perm_b32) and accumulates
//      TB x 8 outputs with v_dot2_f32_bf16 against (o[k], o[k+1]) (exact bf16 products, fp32 sums); the 4 W partials
//      of each output (W waves x 4 lane groups) are summed in LDS in a fixed order;
//   3. the merge_states LSE merge with the window partial (invalid rows zeroed), rounded once to bf16. The window
//      partial of a thread's merge item is loaded at the start, with the split partials.

struct EpilogueParams {
  int T, S;
  const float* ws_o;     // [T][S][16][R] (S > 1)
  const float* ws_lse;   // [T][S][16]
  const uint16_t* o_hist;  // [T][16][R] bf16 (S == 1)
  const float* lse_hist;   // [16][T] (S == 1)
  const uint16_t* B;
  int64_t b_sh, b_sr;
  const uint16_t* o_win;   // [T][16][128]
  const float* lse_win;    // [16][T]
  const uint8_t* invalid;
  uint16_t* out;
  int64_t o_st, o_sh;
};

// Slots whose lse the epilogue stages in LDS: all of them with one token per workgroup, 256 with four.
template <int TB>
constexpr int kEpiSlots = TB == 1 ? kMaxSplits : 256;

template <int R, int TB, int W>
__global__ __launch_bounds__(64 * W) void decode_epilogue(EpilogueParams a) {
  constexpr int kThreads = 64 * W;  // W waves
  constexpr int D = kExactDim, C4 = R / 4;
  constexpr int ITEMS = TB * C4;                               // combine items (token, 4 columns)
  constexpr int IPT = ITEMS > kThreads ? ITEMS / kThreads : 1;  // items per thread
  constexpr int SG = ITEMS < kThreads ? kThreads / ITEMS : 1;   // slot groups: threads sharing one item's slots
  constexpr int RW = R / W;                                    // B rows per wave in the GEMV
  constexpr int NB = RW / 8;                                   // GEMV steps: two B rows per lane each
  constexpr int PB = NB <= 16 ? NB : 0;                        // steps whose rows are prefetched into registers
  static_assert(ITEMS % kThreads == 0 || kThreads % ITEMS == 0, "items must tile the workgroup");
  static_assert(TB * D / 2 <= kThreads, "one merge item per thread");
  __shared__ uint32_t o_s[TB][R / 2];  // bf16 pairs
  __shared__ float lse_s[TB];
  __shared__ floatx4 part[4 * W][TB][D / 4];
  __shared__ float slot_lse[TB][kEpiSlots<TB>];  // lse of every slot of the TB tokens for head h
  __shared__ int used_s[TB];
  __shared__ float merge_m[SG > 1 ? SG : 1][SG > 1 ? ITEMS : 1], merge_d[SG > 1 ? SG : 1][SG > 1 ? ITEMS : 1];
  __shared__ floatx4 merge_o[SG > 1 ? SG : 1][SG > 1 ? ITEMS : 1];
  const int h = blockIdx.y, t0 = blockIdx.x * TB, tid = threadIdx.x;
  const int S = a.S;
  const int q = tid >> 6, lane = tid & 63, g = lane >> 4, c = lane & 15;
  u32x4 bv[PB > 0 ? PB : 1][2];
  const uint16_t* brow = a.B + (int64_t)h * a.b_sh + (int64_t)(q * RW + 2 * g) * a.b_sr + 8 * c;
  // the window partial of this thread's merge item (token t0 + tid / 64, columns 2 * (tid % 64) and + 1)
  const int m_tb = tid / (D / 2), m_dp = tid % (D / 2), m_t = t0 + m_tb;
  const bool m_live = tid < TB * D / 2 && m_t < a.T;
  float w_lse = -INFINITY;
  uint32_t w_o = 0u;
  bool w_inv = false;
  if (m_live) {
    w_lse = a.lse_win[(int64_t)h * a.T + m_t];
    w_o = *reinterpret_cast<const uint32_t*>(a.o_win + ((int64_t)m_t * kHeads + h) * D + 2 * m_dp);
    w_inv = a.invalid && a.invalid[m_t];
  }

  // 1. history output of the TB tokens. Every load of the phase is issued before the first wait: the split
  //    partials and their lse (an empty split left no partial; a select drops it, so its bytes never matter),
  //    then this lane's B rows for the GEMV; the splits are reduced online in chunks of eight (with one token per
  //    workgroup, which meets many slots, each chunk's loads are issued before the previous chunk is reduced).
  if (S > 1) {
    // Round one issues, before any wait: the lse of every slot of the TB tokens (into LDS), the first slots'
    // partials whatever the plan (an unused slot holds lse = -inf and is dropped by a select), and this lane's B
    // rows. The used slots of a row are a prefix (finite lse), so the LDS copy gives their count; only slots past
    // the first round wait for it. Thread groups of SG share one item's slots (slot sg, sg + SG, ...).
    const int sg = SG > 1 ? tid / ITEMS : 0;
    for (int k = tid; k < TB * S; k += kThreads) {
      const int tb = k / S, sl = k % S, t = t0 + tb;
      slot_lse[tb][sl] = t < a.T ? a.ws_lse[((int64_t)t * S + sl) * kHeads + h] : -INFINITY;
    }
    float m[IPT], den[IPT];
    floatx4 acc[IPT];
#pragma unroll
    for (int it = 0; it < IPT; ++it) {
      m[it] = -INFINITY;
      den[it] = 0.f;
      acc[it] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    float ls[IPT][8], ls2[IPT][8];  // two register sets: a round in flight while the previous one is reduced
    floatx4 o[IPT][8], o2[IPT][8];
    auto load_to = [&](int s0, const int (&lim)[IPT], float (&ls)[IPT][8], floatx4 (&o)[IPT][8]) {
      // slots s0 + sg + SG*u, u < 8
#pragma unroll
      for (int it = 0; it < IPT; ++it) {
        const int item = (SG > 1 ? tid % ITEMS : tid) + it * kThreads, tb = item / C4, c4 = item % C4, t = t0 + tb;
        const bool ok = t < a.T;
        const int64_t row = ((int64_t)t * S) * kHeads + h;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int sl = s0 + sg + SG * u;
          const bool use = ok && sl < lim[it];
          ls[it][u] = use ? a.ws_lse[row + (int64_t)sl * kHeads] : -INFINITY;
          o[it][u] = use ? *reinterpret_cast<const floatx4*>(a.ws_o + (row + (int64_t)sl * kHeads) * R + 4 * c4)
                         : floatx4{0.f, 0.f, 0.f, 0.f};
        }
      }
    };
    auto load = [&](int s0, const int (&lim)[IPT]) { load_to(s0, lim, ls, o); };
    // online LSE combine of the eight loaded slots
    auto reduce_from = [&](const float (&ls)[IPT][8], const floatx4 (&o)[IPT][8]) {
#pragma unroll
      for (int it = 0; it < IPT; ++it) {
        float mx = m[it];
#pragma unroll
        for (int u = 0; u < 8; ++u) mx = fmaxf(mx, ls[it][u]);
        if (mx == -INFINITY) continue;
        const float scale = __expf(m[it] - mx);  // 0 while m == -inf
        den[it] *= scale;
        acc[it] = acc[it] * scale;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float w = ls[it][u] == -INFINITY ? 0.f : __expf(ls[it][u] - mx);
          den[it] += w;
          acc[it] += ls[it][u] == -INFINITY ? floatx4{0.f, 0.f, 0.f, 0.f} : o[it][u] * w;
        }
        m[it] = mx;
      }
    };
    {
      int all[IPT];
#pragma unroll
      for (int it = 0; it < IPT; ++it) all[it] = S;
      load(0, all);
    }
#pragma unroll
    for (int step = 0; step < PB; ++step) {
      bv[step][0] = ld16(brow + (int64_t)(8 * step) * a.b_sr);
      bv[step][1] = ld16(brow + (int64_t)(8 * step + 1) * a.b_sr);
    }
    if (tid < TB) used_s[tid] = S;
    __syncthreads();
    // a token's used slots end at its first slot with lse = -inf: every thread checks its slots for that boundary
    // (a serial scan was one dependent LDS read per used slot)
    for (int k = tid; k < TB * S; k += kThreads) {
      const int tb = TB == 1 ? 0 : k / S, sl = k - tb * S;
      if (slot_lse[tb][sl] == -INFINITY && (sl == 0 || slot_lse[tb][sl - 1] != -INFINITY)) atomicMin(&used_s[tb], sl);
    }
    __syncthreads();
    int used[IPT];
    int s_end = 0;
#pragma unroll
    for (int it = 0; it < IPT; ++it) {
      const int tb = ((SG > 1 ? tid % ITEMS : tid) + it * kThreads) / C4;
      used[it] = used_s[tb];
      s_end = max(s_end, used[it]);
    }
    if constexpr (TB == 1) {  // many slots per token: each round's loads are in flight while the previous one is
                              // reduced (same rounds, same order)
      int s0 = 8 * SG;
      if (s0 < s_end) load_to(s0, used, ls2, o2);
      reduce_from(ls, o);
      while (s0 < s_end) {
        const int s1 = s0 + 8 * SG;
        if (s1 < s_end) load_to(s1, used, ls, o);
        reduce_from(ls2, o2);
        if (s1 >= s_end) break;
        const int s2 = s1 + 8 * SG;
        if (s2 < s_end) load_to(s2, used, ls2, o2);
        reduce_from(ls, o);
        s0 = s2;
      }
    } else {
      reduce_from(ls, o);
      for (int s0 = 8 * SG; s0 < s_end; s0 += 8 * SG) {
        load(s0, used);
        reduce_from(ls, o);
      }
    }
    if constexpr (SG > 1) {  // merge the slot groups' partial reductions
      const int item = tid % ITEMS;
      merge_m[sg][item] = m[0];
      merge_d[sg][item] = den[0];
      merge_o[sg][item] = acc[0];
      __syncthreads();
      if (sg == 0) {
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < SG; ++k) mx = fmaxf(mx, merge_m[k][item]);
        float dd = 0.f;
        floatx4 oo = {0.f, 0.f, 0.f, 0.f};
        if (mx != -INFINITY) {
#pragma unroll
          for (int k = 0; k < SG; ++k) {
            const float w = merge_m[k][item] == -INFINITY ? 0.f : __expf(merge_m[k][item] - mx);
            dd += merge_d[k][item] * w;
            oo += merge_o[k][item] * w;
          }
        }
        m[0] = mx;
        den[0] = dd;
        acc[0] = oo;
      }
    }
#pragma unroll
    for (int it = 0; it < IPT; ++it) {
      const int item = tid + it * kThreads;
      if (item >= ITEMS) continue;  // slot groups past the first have merged into it
      const int tb = item / C4, c4 = item % C4;
      const floatx4 o = m[it] == -INFINITY ? floatx4{0.f, 0.f, 0.f, 0.f} : acc[it] * (1.0f / den[it]);
      o_s[tb][2 * c4] = pack2(o[0], o[1]);
      o_s[tb][2 * c4 + 1] = pack2(o[2], o[3]);
      if (c4 == 0) lse_s[tb] = m[it] == -INFINITY ? -INFINITY : m[it] + logf(den[it]);
    }
  } else {
#pragma unroll
    for (int step = 0; step < PB; ++step) {
      bv[step][0] = ld16(brow + (int64_t)(8 * step) * a.b_sr);
      bv[step][1] = ld16(brow + (int64_t)(8 * step + 1) * a.b_sr);
    }
    if (tid < TB) lse_s[tid] = t0 + tid < a.T ? a.lse_hist[(int64_t)h * a.T + t0 + tid] : -INFINITY;
    for (int item = tid; item < TB * R / 2; item += kThreads) {
      const int tb = item / (R / 2), c2 = item % (R / 2), t = t0 + tb;
      o_s[tb][c2] = t < a.T ? *reinterpret_cast<const uint32_t*>(a.o_hist + ((int64_t)t * kHeads + h) * R + 2 * c2)
                            : 0u;
    }
  }
  __syncthreads();

  // 2. GEMV with B[h]
  {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    float acc[TB][8];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[tb][e] = 0.f;
#pragma unroll
    for (int step = 0; step < NB; ++step) {
      const u32x4 b0 = PB > 0 ? bv[step < PB ? step : 0][0] : ld16(brow + (int64_t)(8 * step) * a.b_sr);
      const u32x4 b1 = PB > 0 ? bv[step < PB ? step : 0][1] : ld16(brow + (int64_t)(8 * step + 1) * a.b_sr);
      uint32_t bp[8];  // (B[k][col], B[k + 1][col]) for the lane's 8 columns
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bp[2 * e] = __builtin_amdgcn_perm(b1[e], b0[e], 0x05040100u);
        bp[2 * e + 1] = __builtin_amdgcn_perm(b1[e], b0[e], 0x07060302u);
      }
      const int k2 = (q * RW + 8 * step + 2 * g) / 2;
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        const bf16x2_t o = __builtin_bit_cast(bf16x2_t, o_s[tb][k2]);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          acc[tb][e] = __builtin_amdgcn_fdot2_f32_bf16(o, __builtin_bit_cast(bf16x2_t, bp[e]), acc[tb][e], false);
      }
    }
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      part[q * 4 + g][tb][2 * c] = floatx4{acc[tb][0], acc[tb][1], acc[tb][2], acc[tb][3]};
      part[q * 4 + g][tb][2 * c + 1] = floatx4{acc[tb][4], acc[tb][5], acc[tb][6], acc[tb][7]};
    }
  }
  __syncthreads();

  // 3. merge with the window partial: one item (token, column pair) per thread
  if (m_live) {
    const int tb = m_tb, dp = m_dp, t = m_t;
    float y0 = 0.f, y1 = 0.f;
    const float* pf = reinterpret_cast<const float*>(&part[0][tb][0]) + 2 * dp;
#pragma unroll
    for (int p = 0; p < 4 * W; ++p) {
      y0 += pf[p * TB * D];
      y1 += pf[p * TB * D + 1];
    }
    float lx = lse_s[tb], lb = w_lse;
    if (lx == INFINITY) lx = -INFINITY;  // +inf lse counts as empty
    if (lb == INFINITY) lb = -INFINITY;
    float peak = fmaxf(lx, lb);
    if (isinf(peak)) peak = 0.f;
    float wx = expf(lx - peak), wb = expf(lb - peak);
    const float total = wx + wb;
    if (total > 0.f) {
      wx /= total;
      wb /= total;
    } else {
      wx = wb = 0.f;
    }
    const uint32_t ow = w_o;
    uint32_t res = pack2(rbf(y0) * wx + lo_bf(ow) * wb, rbf(y1) * wx + hi_bf(ow) * wb);
    if (w_inv) res = 0u;
    *reinterpret_cast<uint32_t*>(a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh + 2 * dp) = res;
  }
}

template <int R>
int launch_epilogue(const EpilogueParams& e, hipStream_t stream) {
  // small steps: one token per workgroup, 16*T workgroups for the reduction; with at most 8 tokens (128 or fewer
  // workgroups, fewer than the CUs) 8 waves each, twice the slots per round of loads and half the B rows per wave
  // (B=8 at context 32768: 393.1 -> 389.6 us/layer; B=1: 41.5 -> 39.3 us per call; at 12 and 32 tokens, where two
  // 8-wave workgroups no longer fit a CU beside each other, slower: 183.3 -> 185.4 and 295.1 -> 316.5 us/layer)
  if ((e.T < 64 || e.S > kEpiSlots<4>) && e.T <= 8)
    hipLaunchKernelGGL((decode_epilogue<R, 1, 8>), dim3((unsigned)e.T, kHeads), dim3(512), 0, stream, e);
  else if (e.T < 64 || e.S > kEpiSlots<4>)
    hipLaunchKernelGGL((decode_epilogue<R, 1, 4>), dim3((unsigned)e.T, kHeads), dim3(256), 0, stream, e);
  else
    hipLaunchKernelGGL((decode_epilogue<R, 4, 4>), dim3((unsigned)((e.T + 3) / 4), kHeads), dim3(256), 0, stream, e);
  return check_launch("decode_epilogue");
}

template <int R>
int launch_combine(const HistoryParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(history_combine<R>, dim3(p.T, kHeads), dim3(combine_threads<R>()), 0, stream, p);
  return check_launch("history_combine");
}

// CUs of the current device (256 if the runtime cannot say)
inline int current_device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

// history_mq5 on a grid of (token groups, slots): at R = 256 two tokens per wave when the grid outnumbers the CUs
template <int R, int kMode>
void launch_mq5(const HistoryParams& p, unsigned groups, unsigned slots, hipStream_t stream) {
  const dim3 grid(groups, slots);
  if constexpr (R == 256) {
    if ((uint64_t)groups * slots > (uint64_t)current_device_cus()) {
      hipLaunchKernelGGL((history_mq5<256, kMode, 2>), grid, dim3(64 * Mq5Geo<256, 2>::NW), 0, stream, p);
      return;
    }
  }
  hipLaunchKernelGGL((history_mq5<R, kMode, 1>), grid, dim3(64 * Mq5Geo<R, 1>::NW), 0, stream, p);
}

template <int R>
int launch(const HistoryParams& p, hipStream_t stream) {
  if (p.group > 1) {
    const dim3 grid((unsigned)((p.T + p.group - 1) / p.group), p.num_splits);
    if (p.group == 4 && (R == 256 || R == 512) && p.scale_log2 > 0.f)  // history_mq5 folds a positive scale
      launch_mq5<R == 256 ? 256 : 512, 0>(p, (unsigned)((p.T + kMq4Tokens - 1) / kMq4Tokens), p.num_splits, stream);
    else if (p.group == 4 && R <= 512)
      hipLaunchKernelGGL((history_mq2<R <= 512 ? R : 512, false>), grid, dim3(512), 0, stream, p);
    else  // two tokens per workgroup (four 1024-wide tokens would spill registers and run twice as slow)
      hipLaunchKernelGGL((history_group<R, 2>), dim3((unsigned)((p.T + 1) / 2), p.num_splits), dim3(Geo<R>::THREADS),
                         0, stream, p);
  } else {
    const dim3 grid(split_workgroups(p.T, p.num_splits) + (p.has_window ? window_workgroups(p.T, Geo<R>::WAVES) : 0u));
    if (p.shared_rows) hipLaunchKernelGGL((history_split<R, false>), grid, dim3(Geo<R>::THREADS), 0, stream, p);
    else hipLaunchKernelGGL((history_split<R, true>), grid, dim3(Geo<R>::THREADS), 0, stream, p);
  }
  int rc = check_launch("history_split");
  if (rc == HLA_S6_OK && !p.direct && p.combine) rc = launch_combine<R>(p, stream);
  return rc;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int fill_history(HistoryParams& p, const void* q, int32_t num_tokens, int32_t num_heads, int32_t width, int64_t q_st,
                 int64_t q_sh, const void* k_cache, const void* v_cache, int64_t page_stride, int64_t row_stride,
                 int32_t block_size, int64_t num_blocks, const int32_t* block_table, int64_t bt_stride,
                 int32_t bt_cols, const int64_t* bt_rows, const int32_t* ctx, float scale, int32_t num_splits,
                 float* workspace, int64_t workspace_floats, void* out, int64_t o_st,
                 int64_t o_sh, float* lse, bool partials_only = false) {
  HLA_REQUIRE(num_tokens >= 0, HLA_S6_EINVAL, "history_attention: negative token count");
  HLA_REQUIRE(num_heads == kHeads, HLA_S6_EUNSUPPORTED,
              "history_attention: %d query heads (the kernel is built for 16)", num_heads);
  HLA_REQUIRE(width == 128 || width == 256 || width == 512 || width == 1024, HLA_S6_EUNSUPPORTED,
              "history_attention: latent width %d not in {128, 256, 512, 1024}", width);
  HLA_REQUIRE(block_size > 0 && block_size % kTile == 0, HLA_S6_EUNSUPPORTED,
              "history_attention: block size %d is not a positive multiple of 16", block_size);
  HLA_REQUIRE(num_splits >= 1 && num_splits <= kMaxSplits, HLA_S6_EINVAL,
              "history_attention: num_kv_splits must be in [1, %d]", kMaxSplits);
  HLA_REQUIRE(num_blocks >= 1 && bt_cols >= 0, HLA_S6_EINVAL, "history_attention: empty cache or bad table width");
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(q && k_cache && v_cache && block_table && ctx && (partials_only || (out && lse)), HLA_S6_EINVAL,
              "history_attention: null pointer argument");
  HLA_REQUIRE(aligned16(q) && q_st % 8 == 0 && q_sh % 8 == 0, HLA_S6_EINVAL,
              "history_attention: q needs 16-byte aligned rows (unit last stride, strides multiple of 8)");
  HLA_REQUIRE(aligned16(k_cache) && aligned16(v_cache) && page_stride % 8 == 0 && row_stride % 8 == 0, HLA_S6_EINVAL,
              "history_attention: cache rows must be 16-byte aligned (strides multiple of 8 elements)");
  HLA_REQUIRE((reinterpret_cast<uintptr_t>(out) & 7u) == 0 && o_st % 4 == 0 && o_sh % 4 == 0, HLA_S6_EINVAL,
              "history_attention: output rows must be 8-byte aligned");
  if (num_splits > 1 || partials_only) {
    const int64_t need = (int64_t)num_tokens * num_splits * kHeads * (width + 1);
    HLA_REQUIRE(workspace != nullptr && workspace_floats >= need, HLA_S6_EWORKSPACE,
                "S6 workspace overflow: need %lld floats, have %lld", (long long)need, (long long)workspace_floats);
    HLA_REQUIRE(aligned16(workspace), HLA_S6_EINVAL, "history_attention: workspace must be 16-byte aligned");
  }
  p = HistoryParams{};
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
  p.plan = nullptr;
  p.group = 1;
  p.shared_rows = false;
  p.direct = num_splits == 1 && !partials_only;
  p.combine = !partials_only;
  return HLA_S6_OK;
}

int dispatch(const HistoryParams& p, int width, hipStream_t st) {
  switch (width) {
    case 128: return launch<128>(p, st);
    case 256: return launch<256>(p, st);
    case 512: return launch<512>(p, st);
    default: return launch<1024>(p, st);
  }
}

int dispatch_combine(const HistoryParams& p, int width, hipStream_t st) {
  switch (width) {
    case 128: return launch_combine<128>(p, st);
    case 256: return launch_combine<256>(p, st);
    case 512: return launch_combine<512>(p, st);
    default: return launch_combine<1024>(p, st);
  }
}

}  // namespace
}  // namespace hla

namespace hla {
// Multi-query forward over contiguous rows for the K-hop op (hla_s6_khop_forward): q / z [B * Lq, 16, width]
// (token strides q_st / z_st), k / v [B, N, width] with row stride k_sn (batch stride N * k_sn, N a multiple of
// 16), mask [B, Lq, N] bytes (strides mask_sb, mask_st; mask_st 0 shows one row to all of a batch row's queries)
// or null, bound [B * Lq]. Returns HLA_S6_EUNSUPPORTED when the
// shapes do not fit this kernel or another kernel is faster for them (the caller then uses its own).
int khop_forward_mq(const void* q, int64_t q_st, int64_t q_sh, const void* k, const void* v, int64_t k_sn, int B,
                    int Lq, int N, int width, const uint8_t* mask, int64_t mask_sb, int64_t mask_st,
                    const int32_t* bound, float scale, void* z, int64_t z_st, int64_t z_sh, float* lse,
                    hipStream_t stream) {
  // widths 512 and 256 run faster here than in khop_fwd; history_mq5 takes a positive scale and a mask whose rows
  // start on 16-byte boundaries (its bytes are copied in 16-byte pieces), history_mq2 (width 512) anything else
  const bool mq5 = (width == 512 || width == 256) && scale > 0.f &&
                   (!mask || (((uintptr_t)mask & 15u) == 0 && mask_st % 16 == 0 && mask_sb % 16 == 0));
  if (N % kTile != 0 || (width != 1024 && !(mq5 || width == 512))) return HLA_S6_EUNSUPPORTED;
  HistoryParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.q_st = q_st;
  p.q_sh = q_sh;
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.page_stride = kTile * k_sn;
  p.row_stride = k_sn;
  p.block_size = kTile;
  p.num_blocks = (int64_t)B * (N / kTile);
  p.bt = nullptr;
  p.bt_cols = N / kTile;
  p.tok_per_row = Lq;
  p.ctx = bound;
  p.scale_log2 = scale * kLog2e;
  p.num_splits = 1;
  p.T = B * Lq;
  p.out = static_cast<uint16_t*>(z);
  p.o_st = z_st;
  p.o_sh = z_sh;
  p.lse = lse;
  p.group = kMqTokens;
  p.shared_rows = true;
  p.direct = true;
  p.mask = mask;
  p.mask_st = mask_st;
  p.mask_sb = mask_sb;
  p.mask_split = mask_sb != (int64_t)Lq * mask_st;  // (token-linear rows keep the one-stride form)
  p.reverse_groups = kKhopReverse;
  if (width == 1024) {  // kKhop1024Tokens tokens per workgroup on the 16x16 MFMA group kernel (one wave per 128 columns)
    p.lse_rows = true;
    p.page_stride = (int64_t)N * k_sn;
    hipLaunchKernelGGL((history_group<1024, kKhop1024Tokens, true>),
                       dim3((unsigned)((p.T + kKhop1024Tokens - 1) / kKhop1024Tokens), 1), dim3(Geo<1024>::THREADS), 0,
                       stream, p);
  } else if (mq5) {
    const unsigned groups = (unsigned)((p.T + kMq4Tokens - 1) / kMq4Tokens);
    if (width == 512 && mask) launch_mq5<512, 2>(p, groups, 1, stream);
    else if (width == 512) launch_mq5<512, 1>(p, groups, 1, stream);
    else if (mask) launch_mq5<256, 2>(p, groups, 1, stream);
    else launch_mq5<256, 1>(p, groups, 1, stream);
  } else {
    const dim3 grid((unsigned)((p.T + kMqTokens - 1) / kMqTokens), 1);
    hipLaunchKernelGGL((history_mq2<512, true>), grid, dim3(512), 0, stream, p);
  }
  return check_launch("khop_forward");
}
}  // namespace hla

extern "C" int hla_s6_history_attention(const void* q, int32_t num_tokens, int32_t num_heads, int32_t width,
                                        int64_t q_st, int64_t q_sh, const void* k_cache, const void* v_cache,
                                        int64_t page_stride, int64_t row_stride, int32_t block_size,
                                        int64_t num_blocks, const int32_t* block_table, int64_t bt_stride,
                                        int32_t bt_cols, const int64_t* bt_rows, const int32_t* ctx, float scale,
                                        int32_t num_splits, float* workspace, int64_t workspace_floats, void* out,
                                        int64_t o_st, int64_t o_sh, float* lse,
                                        void* stream) {
  using namespace hla;
  HistoryParams p;
  int rc = fill_history(p, q, num_tokens, num_heads, width, q_st, q_sh, k_cache, v_cache, page_stride, row_stride,
                        block_size, num_blocks, block_table, bt_stride, bt_cols, bt_rows, ctx, scale, num_splits,
                        workspace, workspace_floats, out, o_st, o_sh, lse);
  if (rc != HLA_S6_OK || num_tokens == 0) return rc;
  return dispatch(p, width, as_stream(stream));
}

extern "C" int hla_s6_history_attention_grouped(
    const void* q, int32_t num_tokens, int32_t num_heads, int32_t width, int64_t q_st, int64_t q_sh,
    const void* k_cache, const void* v_cache, int64_t page_stride, int64_t row_stride, int32_t block_size,
    int64_t num_blocks, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols, const int64_t* bt_rows,
    const int32_t* ctx, float scale, int32_t num_splits, float* workspace, int64_t workspace_floats, void* out,
    int64_t o_st, int64_t o_sh, float* lse, int32_t group, int32_t shared_rows, void* stream) {
  using namespace hla;
  HLA_REQUIRE(group == 1 || group == 2 || group == 4, HLA_S6_EUNSUPPORTED,
              "history_attention: group of %d tokens (built for 1, 2, 4)", group);
  HistoryParams p;
  int rc = fill_history(p, q, num_tokens, num_heads, width, q_st, q_sh, k_cache, v_cache, page_stride, row_stride,
                        block_size, num_blocks, block_table, bt_stride, bt_cols, bt_rows, ctx, scale, num_splits,
                        workspace, workspace_floats, out, o_st, o_sh, lse);
  if (rc != HLA_S6_OK || num_tokens == 0) return rc;
  p.group = group;
  p.shared_rows = shared_rows != 0 || group > 1;
  return dispatch(p, width, as_stream(stream));
}

extern "C" int hla_s6_masked_history(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v,
                                     int64_t kv_sb, int64_t kv_sn, const uint8_t* mask, int64_t m_sb,
                                     const int32_t* bound, int32_t B, int32_t N, int32_t num_heads, int32_t width,
                                     float scale, int32_t num_splits, float* workspace, int64_t workspace_floats,
                                     void* z, int64_t z_sb, int64_t z_sh, float* lse, void* stream) {
  using namespace hla;
  HLA_REQUIRE(B >= 0 && N >= 1, HLA_S6_EINVAL, "masked_history: need B >= 0 and at least one storage row");
  HLA_REQUIRE(num_heads == kHeads, HLA_S6_EUNSUPPORTED, "masked_history: %d heads (the kernel is built for 16)",
              num_heads);
  HLA_REQUIRE(width == 128 || width == 256 || width == 512 || width == 1024, HLA_S6_EUNSUPPORTED,
              "masked_history: latent width %d not in {128, 256, 512, 1024}", width);
  HLA_REQUIRE(num_splits >= 1 && num_splits <= kMaxSplits, HLA_S6_EINVAL,
              "masked_history: num_splits must be in [1, %d]", kMaxSplits);
  if (B == 0) return HLA_S6_OK;
  HLA_REQUIRE(q && k && v && bound && z && lse, HLA_S6_EINVAL, "masked_history: null pointer argument");
  HLA_REQUIRE(aligned16(q) && q_sb % 8 == 0 && q_sh % 8 == 0, HLA_S6_EINVAL,
              "masked_history: q needs 16-byte aligned rows (unit last stride, strides multiple of 8)");
  HLA_REQUIRE(aligned16(k) && aligned16(v) && kv_sb % 8 == 0 && kv_sn % 8 == 0, HLA_S6_EINVAL,
              "masked_history: k / v rows must be 16-byte aligned (strides multiple of 8 elements)");
  HLA_REQUIRE((reinterpret_cast<uintptr_t>(z) & 7u) == 0 && z_sb % 4 == 0 && z_sh % 4 == 0, HLA_S6_EINVAL,
              "masked_history: z rows must be 8-byte aligned");
  HLA_REQUIRE(!mask || m_sb >= N, HLA_S6_EINVAL, "masked_history: mask row stride below N");
  if (num_splits > 1) {
    const int64_t need = (int64_t)B * num_splits * kHeads * (width + 1);
    HLA_REQUIRE(workspace != nullptr && workspace_floats >= need, HLA_S6_EWORKSPACE,
                "S6 workspace overflow: need %lld floats, have %lld", (long long)need, (long long)workspace_floats);
    HLA_REQUIRE(aligned16(workspace), HLA_S6_EINVAL, "masked_history: workspace must be 16-byte aligned");
  }
  HistoryParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.q_st = q_sb;
  p.q_sh = q_sh;
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.page_stride = kv_sb;  // one "page" per batch row holding its N rows
  p.row_stride = kv_sn;
  p.block_size = N;
  p.num_blocks = B;
  p.bt = nullptr;
  p.bt_cols = 1;
  p.tok_per_row = 1;
  p.lse_rows = true;
  p.ctx = bound;
  p.mask = mask;
  p.mask_st = m_sb;
  p.scale_log2 = scale * kLog2e;
  p.num_splits = num_splits;
  p.T = B;
  p.ws_o = num_splits > 1 ? workspace : nullptr;
  p.ws_lse = num_splits > 1 ? workspace + (int64_t)B * num_splits * kHeads * width : nullptr;
  p.out = static_cast<uint16_t*>(z);
  p.o_st = z_sb;
  p.o_sh = z_sh;
  p.lse = lse;
  p.group = 1;
  p.direct = num_splits == 1;
  p.combine = true;
  const hipStream_t st = as_stream(stream);
  const dim3 grid(split_workgroups(B, num_splits));
  switch (width) {
    case 128: hipLaunchKernelGGL((history_split<128, true, true>), grid, dim3(Geo<128>::THREADS), 0, st, p); break;
    case 256: hipLaunchKernelGGL((history_split<256, true, true>), grid, dim3(Geo<256>::THREADS), 0, st, p); break;
    case 512: hipLaunchKernelGGL((history_split<512, true, true>), grid, dim3(Geo<512>::THREADS), 0, st, p); break;
    default: hipLaunchKernelGGL((history_split<1024, true, true>), grid, dim3(Geo<1024>::THREADS), 0, st, p); break;
  }
  int rc = check_launch("masked_history");
  if (rc == HLA_S6_OK && num_splits > 1) rc = dispatch_combine(p, width, st);
  return rc;
}

extern "C" int hla_s6_history_partials(const void* q, int32_t num_tokens, int32_t num_heads, int32_t width,
                                       int64_t q_st, int64_t q_sh, const void* k_cache, const void* v_cache,
                                       int64_t page_stride, int64_t row_stride, int32_t block_size, int64_t num_blocks,
                                       const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                                       const int64_t* bt_rows, const int32_t* ctx, float scale, int32_t num_splits,
                                       float* workspace, int64_t workspace_floats, const int32_t* plan,
                                       int64_t plan_len, void* stream) {
  using namespace hla;
  HistoryParams p;
  int rc = fill_history(p, q, num_tokens, num_heads, width, q_st, q_sh, k_cache, v_cache, page_stride, row_stride,
                        block_size, num_blocks, block_table, bt_stride, bt_cols, bt_rows, ctx, scale, num_splits,
                        workspace, workspace_floats, nullptr, 0, 0, nullptr, true);
  if (rc != HLA_S6_OK || num_tokens == 0) return rc;
  if (plan && num_splits > 1) {
    HLA_REQUIRE(plan_len >= plan_ints(num_tokens, num_splits), HLA_S6_EINVAL,
                "history_partials: split plan of %lld ints, need %lld", (long long)plan_len,
                (long long)plan_ints(num_tokens, num_splits));
    p.plan = plan;
  }
  return dispatch(p, width, as_stream(stream));
}

extern "C" int hla_s6_history_partials_grouped(const void* q, int32_t num_tokens, int32_t num_heads, int32_t width,
                                               int64_t q_st, int64_t q_sh, const void* k_cache, const void* v_cache,
                                               int64_t page_stride, int64_t row_stride, int32_t block_size,
                                               int64_t num_blocks, const int32_t* block_table, int64_t bt_stride,
                                               int32_t bt_cols, const int64_t* bt_rows, const int32_t* ctx,
                                               float scale, int32_t num_splits, float* workspace,
                                               int64_t workspace_floats, int32_t group, void* stream) {
  using namespace hla;
  HLA_REQUIRE(group == 2 || group == 4, HLA_S6_EUNSUPPORTED,
              "history_partials_grouped: group of %d tokens (built for 2, 4)", group);
  HistoryParams p;
  int rc = fill_history(p, q, num_tokens, num_heads, width, q_st, q_sh, k_cache, v_cache, page_stride, row_stride,
                        block_size, num_blocks, block_table, bt_stride, bt_cols, bt_rows, ctx, scale, num_splits,
                        workspace, workspace_floats, nullptr, 0, 0, nullptr, true);
  if (rc != HLA_S6_OK || num_tokens == 0) return rc;
  p.group = group;
  p.shared_rows = true;
  return dispatch(p, width, as_stream(stream));
}

extern "C" int hla_s6_split_epilogue(const float* workspace, int64_t workspace_floats, int32_t num_tokens,
                                     int32_t num_heads, int32_t width, int32_t num_splits, const void* B, int64_t b_sh,
                                     int64_t b_sr, const void* o_win, const float* lse_win, const uint8_t* invalid,
                                     void* out, int64_t o_st, int64_t o_sh, void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_tokens >= 0, HLA_S6_EINVAL, "split_epilogue: negative token count");
  HLA_REQUIRE(num_heads == kHeads, HLA_S6_EUNSUPPORTED, "split_epilogue: %d query heads (the kernel is built for 16)",
              num_heads);
  HLA_REQUIRE(width == 128 || width == 256 || width == 512 || width == 1024, HLA_S6_EUNSUPPORTED,
              "split_epilogue: latent width %d not in {128, 256, 512, 1024}", width);
  HLA_REQUIRE(num_splits >= 2 && num_splits <= kMaxSplits, HLA_S6_EINVAL,
              "split_epilogue: num_kv_splits must be in [2, %d]", kMaxSplits);
  if (num_tokens == 0) return HLA_S6_OK;
  const int64_t need = (int64_t)num_tokens * num_splits * kHeads * (width + 1);
  HLA_REQUIRE(workspace != nullptr && workspace_floats >= need, HLA_S6_EWORKSPACE,
              "S6 workspace overflow: need %lld floats, have %lld", (long long)need, (long long)workspace_floats);
  HLA_REQUIRE(aligned16(workspace), HLA_S6_EINVAL, "split_epilogue: workspace must be 16-byte aligned");
  HLA_REQUIRE(B && o_win && lse_win && out, HLA_S6_EINVAL, "split_epilogue: null pointer argument");
  HLA_REQUIRE(aligned16(o_win), HLA_S6_EINVAL, "split_epilogue: o_win must be 16-byte aligned");
  HLA_REQUIRE((reinterpret_cast<uintptr_t>(B) & 3u) == 0 && b_sh % 2 == 0 && b_sr % 2 == 0 &&
                  (reinterpret_cast<uintptr_t>(out) & 3u) == 0 && o_st % 2 == 0 && o_sh % 2 == 0,
              HLA_S6_EINVAL, "split_epilogue: B and out need 4-byte aligned pairs");
  EpilogueParams e = {};
  e.T = num_tokens;
  e.S = num_splits;
  e.ws_o = workspace;
  e.ws_lse = workspace + (int64_t)num_tokens * num_splits * kHeads * width;
  e.B = static_cast<const uint16_t*>(B);
  e.b_sh = b_sh;
  e.b_sr = b_sr;
  e.o_win = static_cast<const uint16_t*>(o_win);
  e.lse_win = lse_win;
  e.invalid = invalid;
  e.out = static_cast<uint16_t*>(out);
  e.o_st = o_st;
  e.o_sh = o_sh;
  const hipStream_t st = as_stream(stream);
  switch (width) {
    case 128: return launch_epilogue<128>(e, st);
    case 256: return launch_epilogue<256>(e, st);
    case 512: return launch_epilogue<512>(e, st);
    default: return launch_epilogue<1024>(e, st);
  }
}

extern "C" int hla_s6_history_reduce(const float* workspace, int64_t workspace_floats, int32_t num_tokens,
                                     int32_t num_heads, int32_t width, int32_t num_splits, void* out, int64_t o_st,
                                     int64_t o_sh, float* lse, void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_tokens >= 0, HLA_S6_EINVAL, "history_reduce: negative token count");
  HLA_REQUIRE(num_heads == kHeads, HLA_S6_EUNSUPPORTED,
              "history_reduce: %d query heads (the kernel is built for 16)", num_heads);
  HLA_REQUIRE(width == 128 || width == 256 || width == 512 || width == 1024, HLA_S6_EUNSUPPORTED,
              "history_reduce: latent width %d not in {128, 256, 512, 1024}", width);
  HLA_REQUIRE(num_splits >= 1 && num_splits <= kMaxSplits, HLA_S6_EINVAL,
              "history_reduce: num_kv_splits must be in [1, %d]", kMaxSplits);
  if (num_tokens == 0) return HLA_S6_OK;
  const int64_t need = (int64_t)num_tokens * num_splits * kHeads * (width + 1);
  HLA_REQUIRE(workspace != nullptr && workspace_floats >= need, HLA_S6_EWORKSPACE,
              "S6 workspace overflow: need %lld floats, have %lld", (long long)need, (long long)workspace_floats);
  HLA_REQUIRE(aligned16(workspace), HLA_S6_EINVAL, "history_reduce: workspace must be 16-byte aligned");
  HLA_REQUIRE(out && lse, HLA_S6_EINVAL, "history_reduce: null pointer argument");
  HLA_REQUIRE((reinterpret_cast<uintptr_t>(out) & 7u) == 0 && o_st % 4 == 0 && o_sh % 4 == 0, HLA_S6_EINVAL,
              "history_reduce: output rows must be 8-byte aligned");
  HistoryParams p = {};
  p.num_splits = num_splits;
  p.T = num_tokens;
  p.ws_o = const_cast<float*>(workspace);
  p.ws_lse = p.ws_o + (int64_t)num_tokens * num_splits * kHeads * width;
  p.out = static_cast<uint16_t*>(out);
  p.o_st = o_st;
  p.o_sh = o_sh;
  p.lse = lse;
  return dispatch_combine(p, width, as_stream(stream));
}

extern "C" int64_t hla_s6_split_plan_ints(int32_t num_tokens, int32_t num_splits) {
  return num_tokens < 0 || num_splits < 1 ? -1 : hla::plan_ints(num_tokens, num_splits);
}

extern "C" int hla_s6_split_plans(const int32_t* ctx, int32_t num_tokens, int64_t cap, int32_t count,
                                  const int32_t* num_splits, const int32_t* query_start_loc, int32_t num_reqs,
                                  int32_t* const* plans, const int64_t* plan_lens, void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_tokens >= 0 && cap >= 0 && count >= 1 && count <= kMaxPlans, HLA_S6_EINVAL,
              "split_plans: bad token count, key capacity or plan count (1..%d)", kMaxPlans);
  HLA_REQUIRE(num_splits && plans && plan_lens, HLA_S6_EINVAL, "split_plans: null host array");
  PlanSet set{};
  for (int i = 0; i < count; ++i) {
    HLA_REQUIRE(num_splits[i] >= 1 && num_splits[i] <= kMaxSplits, HLA_S6_EINVAL,
                "split_plans: slot count %d outside 1..%d", num_splits[i], kMaxSplits);
    HLA_REQUIRE(num_tokens == 0 || plans[i], HLA_S6_EINVAL, "split_plans: null plan %d", i);
    HLA_REQUIRE(plan_lens[i] >= plan_ints(num_tokens, num_splits[i]), HLA_S6_EINVAL,
                "split_plans: plan %d has %lld ints, needs %lld", i, (long long)plan_lens[i],
                (long long)plan_ints(num_tokens, num_splits[i]));
    set.S[i] = num_splits[i];
    set.plan[i] = plans[i];
  }
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(ctx, HLA_S6_EINVAL, "split_plans: null ctx");
  HLA_REQUIRE(!query_start_loc || num_reqs >= 1, HLA_S6_EINVAL, "split_plans: query_start_loc needs num_reqs >= 1");
  hipLaunchKernelGGL(split_plan_kernel, dim3((unsigned)count), dim3(256), 0, as_stream(stream), ctx, num_tokens, cap,
                     set, query_start_loc, num_reqs);
  return check_launch("split_plans");
}

extern "C" int hla_s6_split_plan(const int32_t* ctx, int32_t num_tokens, int64_t cap, int32_t num_splits,
                                 const int32_t* query_start_loc, int32_t num_reqs, int32_t* plan, int64_t plan_len,
                                 void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_tokens >= 0 && num_splits >= 1 && num_splits <= kMaxSplits && cap >= 0, HLA_S6_EINVAL,
              "split_plan: bad token count, slot count or key capacity");
  if (num_tokens == 0) return HLA_S6_OK;
  HLA_REQUIRE(ctx && plan, HLA_S6_EINVAL, "split_plan: null pointer argument");
  HLA_REQUIRE(plan_len >= plan_ints(num_tokens, num_splits), HLA_S6_EINVAL, "split_plan: %lld ints, need %lld",
              (long long)plan_len, (long long)plan_ints(num_tokens, num_splits));
  HLA_REQUIRE(!query_start_loc || num_reqs >= 1, HLA_S6_EINVAL, "split_plan: query_start_loc needs num_reqs >= 1");
  PlanSet set{};
  set.S[0] = num_splits;
  set.plan[0] = plan;
  hipLaunchKernelGGL(split_plan_kernel, dim3(1), dim3(256), 0, as_stream(stream), ctx, num_tokens, cap, set,
                     query_start_loc, num_reqs);
  return check_launch("split_plan");
}

namespace hla {
namespace {
// The fused decode attention of one layer x loop behind hla_s6_attend_decode and hla_s6_attend_decode_static.
int attend_decode(
    const void* q_lat, int64_t ql_st, int64_t ql_sh, int32_t width, const void* lat_k, const void* lat_v,
    int64_t lat_page_stride, int64_t lat_row_stride, int32_t block_size, int64_t lat_num_blocks,
    const int32_t* lat_table, int64_t lat_bt_stride, int32_t lat_bt_cols, const int64_t* token_requests,
    const int32_t* ctx_latent, const void* q_rope, int64_t qr_st, int64_t qr_sh, const void* ex_k, const void* ex_v,
    int64_t ex_page_stride, int64_t ex_row_stride, int64_t ex_head_stride, int32_t ex_block_size,
    int64_t ex_num_blocks, const int32_t* ex_table, int64_t ex_bt_stride, int32_t ex_bt_cols,
    const int32_t* query_start_loc, const int32_t* seq_lens, int32_t num_reqs, int32_t window, const void* B,
    int64_t b_sh, int64_t b_sr, const uint8_t* invalid, int32_t num_tokens, int32_t num_heads, float scale,
    int32_t num_splits, int32_t max_query_len, float* workspace, int64_t workspace_floats, const int32_t* plan,
    int64_t plan_len, void* o_hist, float* lse_hist, void* o_win, float* lse_win, void* out, int64_t o_st,
    int64_t o_sh, hipStream_t st) {
  HistoryParams p;
  int rc = fill_history(p, q_lat, num_tokens, num_heads, width, ql_st, ql_sh, lat_k, lat_v, lat_page_stride,
                        lat_row_stride, block_size, lat_num_blocks, lat_table, lat_bt_stride, lat_bt_cols,
                        token_requests, ctx_latent, scale, num_splits, workspace, workspace_floats, o_hist,
                        (int64_t)num_heads * width, width, lse_hist);
  if (rc != HLA_S6_OK || num_tokens == 0) return rc;
  HLA_REQUIRE(q_rope && ex_k && ex_v && ex_table && query_start_loc && seq_lens && num_reqs >= 1 && B && o_win &&
                  lse_win && out && token_requests,
              HLA_S6_EINVAL, "attend_decode: null pointer argument");
  HLA_REQUIRE(window >= 0 && ex_block_size > 0 && ex_num_blocks >= 1 && ex_bt_cols >= 0, HLA_S6_EINVAL,
              "attend_decode: bad window, exact block size, cache size or table width");
  HLA_REQUIRE(aligned16(q_rope) && qr_st % 8 == 0 && qr_sh % 8 == 0 && aligned16(ex_k) && aligned16(ex_v) &&
                  ex_page_stride % 8 == 0 && ex_row_stride % 8 == 0 && ex_head_stride % 8 == 0 && aligned16(o_win),
              HLA_S6_EINVAL, "attend_decode: exact rows must be 16-byte aligned");
  p.has_window = true;
  WindowPart& w = p.win;
  w.src.k = static_cast<const uint16_t*>(ex_k);
  w.src.v = static_cast<const uint16_t*>(ex_v);
  w.src.paged = true;
  w.src.page_stride = ex_page_stride;
  w.src.row_stride = ex_row_stride;
  w.src.head_stride = ex_head_stride;
  w.src.num_blocks = ex_num_blocks;
  w.src.block_size = ex_block_size;
  w.q = static_cast<const uint16_t*>(q_rope);
  w.q_st = qr_st;
  w.q_sh = qr_sh;
  w.bt = ex_table;
  w.bt_stride = ex_bt_stride;
  w.bt_cols = ex_bt_cols;
  w.qsl = query_start_loc;
  w.seq_lens = seq_lens;
  w.num_reqs = num_reqs;
  w.window = window;
  w.chunk_start = true;  // = the decode window for one-token requests; the chunk + window history otherwise
  w.token_requests = token_requests;
  w.out = static_cast<uint16_t*>(o_win);
  w.o_st = (int64_t)num_heads * kExactDim;
  w.o_sh = kExactDim;
  w.lse = lse_win;
  HLA_REQUIRE((reinterpret_cast<uintptr_t>(B) & 3u) == 0 && b_sh % 2 == 0 && b_sr % 2 == 0 &&
                  (reinterpret_cast<uintptr_t>(out) & 3u) == 0 && o_st % 2 == 0 && o_sh % 2 == 0,
              HLA_S6_EINVAL, "attend_decode: B and out need 4-byte aligned pairs");
  if (plan && num_splits > 1) {
    HLA_REQUIRE(plan_len >= plan_ints(num_tokens, num_splits), HLA_S6_EINVAL,
                "attend_decode: split plan of %lld ints, need %lld", (long long)plan_len,
                (long long)plan_ints(num_tokens, num_splits));
    p.plan = plan;
  }
  p.combine = false;  // the epilogue reduces the splits
  p.shared_rows = max_query_len > 1;  // tokens of a chunk read the same rows: cached loads (decode: streaming)
  rc = dispatch(p, width, st);
  if (rc != HLA_S6_OK) return rc;
  EpilogueParams e = {};
  e.T = num_tokens;
  e.S = num_splits;
  e.ws_o = p.ws_o;
  e.ws_lse = p.ws_lse;
  e.o_hist = static_cast<const uint16_t*>(o_hist);
  e.lse_hist = lse_hist;
  e.B = static_cast<const uint16_t*>(B);
  e.b_sh = b_sh;
  e.b_sr = b_sr;
  e.o_win = static_cast<const uint16_t*>(o_win);
  e.lse_win = lse_win;
  e.invalid = invalid;
  e.out = static_cast<uint16_t*>(out);
  e.o_st = o_st;
  e.o_sh = o_sh;
  switch (width) {
    case 128: return launch_epilogue<128>(e, st);
    case 256: return launch_epilogue<256>(e, st);
    case 512: return launch_epilogue<512>(e, st);
    default: return launch_epilogue<1024>(e, st);
  }
}
}  // namespace
}  // namespace hla

extern "C" int hla_s6_attend_decode(
    const void* q_lat, int64_t ql_st, int64_t ql_sh, int32_t width, const void* lat_k, const void* lat_v,
    int64_t lat_page_stride, int64_t lat_row_stride, int32_t block_size, int64_t lat_num_blocks,
    const int32_t* lat_table, int64_t lat_bt_stride, int32_t lat_bt_cols, const int64_t* token_requests,
    const int32_t* ctx_latent, const void* q_rope, int64_t qr_st, int64_t qr_sh, const void* ex_k, const void* ex_v,
    int64_t ex_page_stride, int64_t ex_row_stride, int64_t ex_head_stride, int32_t ex_block_size,
    int64_t ex_num_blocks, const int32_t* ex_table, int64_t ex_bt_stride, int32_t ex_bt_cols,
    const int32_t* query_start_loc, const int32_t* seq_lens, int32_t num_reqs, int32_t window, const void* B,
    int64_t b_sh, int64_t b_sr, const uint8_t* invalid, int32_t num_tokens, int32_t num_heads, float scale,
    int32_t num_splits, int32_t max_query_len, float* workspace, int64_t workspace_floats, const int32_t* plan,
    int64_t plan_len, void* o_hist, float* lse_hist, void* o_win, float* lse_win, void* out, int64_t o_st,
    int64_t o_sh, void* stream) {
  return hla::attend_decode(q_lat, ql_st, ql_sh, width, lat_k, lat_v, lat_page_stride, lat_row_stride, block_size,
                            lat_num_blocks, lat_table, lat_bt_stride, lat_bt_cols, token_requests, ctx_latent, q_rope,
                            qr_st, qr_sh, ex_k, ex_v, ex_page_stride, ex_row_stride, ex_head_stride, ex_block_size,
                            ex_num_blocks, ex_table, ex_bt_stride, ex_bt_cols, query_start_loc, seq_lens, num_reqs,
                            window, B, b_sh, b_sr, invalid, num_tokens, num_heads, scale, num_splits, max_query_len,
                            workspace, workspace_floats, plan, plan_len, o_hist, lse_hist, o_win, lse_win, out, o_st,
                            o_sh, hla::as_stream(stream));
}

// ---- hla_s6_attend_decode_static: the fused decode step with its buffers in a static device array -------------
// For callers that cannot allocate. `scratch` holds, per call, the split partials (T * S * 16 * (width + 1)
// floats), the step's split plan, the history output and lse (written by a one-slot call), and the exact window's
// output and lse, each region 256-byte aligned. Every GPU holds its own copy of the array for the life of the process; its
// address on a device comes from hipGetSymbolAddress with that device current, once per device, and host code uses
// only that address (the array's name is a host-side stand-in). Nothing in it needs clearing: every word a kernel of
// the call reads was written earlier in the same call. Calls that overlap on one GPU share the array and race.
namespace hla {
namespace {
constexpr int64_t kStaticScratchBytes = 48ll << 20;
constexpr int kMaxDevices = 64;
}  // namespace
}  // namespace hla

static __device__ __align__(256) float scratch[hla::kStaticScratchBytes / sizeof(float)];

namespace hla {
namespace {
std::mutex g_scratch_mutex;
void* g_scratch_addr[kMaxDevices] = {};

// This device's copy of `scratch`, looked up on the first call on the device.
int static_scratch(void** addr) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return fail(HLA_S6_EDEVICE, "attend_decode_static: %s", hipGetErrorString(err));
  HLA_REQUIRE(dev >= 0 && dev < kMaxDevices, HLA_S6_EDEVICE, "attend_decode_static: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p)
      return fail(HLA_S6_EDEVICE, "attend_decode_static: no device address for the scratch array: %s",
                  hipGetErrorString(err));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return HLA_S6_OK;
}

inline int64_t align256(int64_t bytes) { return (bytes + 255) / 256 * 256; }
}  // namespace
}  // namespace hla

extern "C" int hla_s6_attend_decode_static(
    const void* q_lat, int64_t ql_st, int64_t ql_sh, int32_t width, const void* lat_k, const void* lat_v,
    int64_t lat_page_stride, int64_t lat_row_stride, int32_t block_size, int64_t lat_num_blocks,
    const int32_t* lat_table, int64_t lat_bt_stride, int32_t lat_bt_cols, const int64_t* token_requests,
    const int32_t* ctx_latent, const void* q_rope, int64_t qr_st, int64_t qr_sh, const void* ex_k, const void* ex_v,
    int64_t ex_page_stride, int64_t ex_row_stride, int64_t ex_head_stride, int32_t ex_block_size,
    int64_t ex_num_blocks, const int32_t* ex_table, int64_t ex_bt_stride, int32_t ex_bt_cols,
    const int32_t* query_start_loc, const int32_t* seq_lens, int32_t num_reqs, int32_t window, const void* B,
    int64_t b_sh, int64_t b_sr, const uint8_t* invalid, int32_t num_tokens, int32_t num_heads, float scale,
    int32_t num_splits, int32_t max_query_len, void* out, int64_t o_st, int64_t o_sh, void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_tokens >= 0 && num_splits >= 1 && num_splits <= kMaxSplits && num_heads == kHeads &&
                  (width == 128 || width == 256 || width == 512 || width == 1024),
              HLA_S6_EINVAL, "attend_decode_static: bad token count, split count, head count or width");
  if (num_tokens == 0) return HLA_S6_OK;
  const int64_t T = num_tokens, S = num_splits;
  const int64_t ws_bytes = S > 1 ? align256(T * S * kHeads * (width + 1) * 4) : 0;
  const int64_t plan_bytes = S > 1 ? align256(plan_ints(num_tokens, num_splits) * 4) : 0;
  const int64_t hist_bytes = align256(T * kHeads * width * 2) + align256(kHeads * T * 4);
  const int64_t win_bytes = align256(T * kHeads * kExactDim * 2) + align256(kHeads * T * 4);
  const int64_t need = ws_bytes + plan_bytes + hist_bytes + win_bytes;
  HLA_REQUIRE(need <= kStaticScratchBytes, HLA_S6_EWORKSPACE,
              "attend_decode_static: %d tokens x %d splits at width %d need %lld scratch bytes, the static array "
              "holds %lld",
              num_tokens, num_splits, width, (long long)need, (long long)kStaticScratchBytes);
  void* base = nullptr;
  int rc = static_scratch(&base);
  if (rc != HLA_S6_OK) return rc;
  char* at = static_cast<char*>(base);
  float* ws = S > 1 ? reinterpret_cast<float*>(at) : nullptr;
  at += ws_bytes;
  int32_t* plan = S > 1 ? reinterpret_cast<int32_t*>(at) : nullptr;
  at += plan_bytes;
  void* o_hist = at;  // written by a one-slot call only, as in hla_s6_attend_decode
  at += align256(T * kHeads * width * 2);
  float* lse_hist = reinterpret_cast<float*>(at);
  at += align256(kHeads * T * 4);
  void* o_win = at;
  at += align256(T * kHeads * kExactDim * 2);
  float* lse_win = reinterpret_cast<float*>(at);
  hipStream_t st = as_stream(stream);
  if (S > 1) {  // the step's split plan into the scratch (one small launch)
    HLA_REQUIRE(ctx_latent && query_start_loc && num_reqs >= 1, HLA_S6_EINVAL,
                "attend_decode_static: null ctx_latent or query_start_loc");
    PlanSet set{};
    set.S[0] = num_splits;
    set.plan[0] = plan;
    hipLaunchKernelGGL(split_plan_kernel, dim3(1), dim3(256), 0, st, ctx_latent, num_tokens,
                       (int64_t)lat_bt_cols * block_size, set, max_query_len > 1 ? query_start_loc : nullptr,
                       num_reqs);
    rc = check_launch("attend_decode_static: split plan");
    if (rc != HLA_S6_OK) return rc;
  }
  return attend_decode(q_lat, ql_st, ql_sh, width, lat_k, lat_v, lat_page_stride, lat_row_stride, block_size,
                       lat_num_blocks, lat_table, lat_bt_stride, lat_bt_cols, token_requests, ctx_latent, q_rope,
                       qr_st, qr_sh, ex_k, ex_v, ex_page_stride, ex_row_stride, ex_head_stride, ex_block_size,
                       ex_num_blocks, ex_table, ex_bt_stride, ex_bt_cols, query_start_loc, seq_lens, num_reqs, window,
                       B, b_sh, b_sr, invalid, num_tokens, num_heads, scale, num_splits, max_query_len, ws,
                       S > 1 ? ws_bytes / 4 : 0, plan, S > 1 ? plan_ints(num_tokens, num_splits) : 0, o_hist,
                       lse_hist, o_win, lse_win, out, o_st, o_sh, st);
}
