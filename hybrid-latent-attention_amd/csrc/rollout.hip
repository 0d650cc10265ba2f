// Rollout-cache gather: one request's committed latent rows of every layer, read through its block lists from
// the paged main and loop-1 caches and packed as [layers, length, 2r + 2r1] rows
// ([main K | main V | loop-1 K | loop-1 V], the packed row of hla/latent/register.py:73-79), in one launch.
// This is the device half of the s6-rollout-cache-v1 export (hla/vllm_latent/cache_export.py:159-188), which
// gathers `cache[block[pos // block_size], 0, pos % block_size, :]` per layer and cache and concatenates.
//
// A workgroup moves 4 rows of one layer; 64 threads per row copy 16-byte pieces when every row and stride allows
// it, single elements otherwise. Pure data movement: HBM-bound, 2 x length x (2r + 2r1) x 2 bytes per layer.
#include "common.h"

namespace hla {
namespace {

struct PackParams {
  const int64_t* addrs;  // [2 * layers] device addresses: main cache of layer l at 2l, loop-1 cache at 2l + 1
  int layers, length;
  int64_t page_stride[2], row_stride[2], num_blocks[2];
  int width2[2];  // elements per cache row (2r, 2r1)
  const int32_t* blocks[2];
  int block_size[2];
  uint16_t* out;
  int64_t out_layer_stride, out_row_stride;
};

template <bool VEC>
__global__ __launch_bounds__(256) void pack_rows_kernel(PackParams a) {
  const int layer = blockIdx.y;
  const int pos = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (pos >= a.length) return;
  uint16_t* dst = a.out + (int64_t)layer * a.out_layer_stride + (int64_t)pos * a.out_row_stride;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int64_t block = a.blocks[c][pos / a.block_size[c]];
    const int w2 = a.width2[c];
    uint16_t* d = dst + (c == 0 ? 0 : a.width2[0]);
    const bool ok = block >= 0 && block < a.num_blocks[c];
    const uint16_t* src = reinterpret_cast<const uint16_t*>(a.addrs[2 * layer + c]) +
                          (ok ? block * a.page_stride[c] + (int64_t)(pos % a.block_size[c]) * a.row_stride[c] : 0);
    if (VEC) {
      for (int i = lane; i < w2 / 8; i += 64)
        st16(d + 8 * i, ok ? ld16(src + 8 * i) : u32x4{0u, 0u, 0u, 0u});
    } else {
      for (int i = lane; i < w2; i += 64) d[i] = ok ? src[i] : (uint16_t)0;
    }
  }
}

}  // namespace
}  // namespace hla

extern "C" int hla_s6_gather_packed_rows(const int64_t* cache_addrs, int32_t num_layers, int64_t main_page_stride,
                                         int64_t main_row_stride, int32_t main_width, int64_t main_num_blocks,
                                         const int32_t* main_blocks, int32_t main_block_size,
                                         int64_t l1_page_stride, int64_t l1_row_stride, int32_t l1_width,
                                         int64_t l1_num_blocks, const int32_t* l1_blocks, int32_t l1_block_size,
                                         int32_t length, void* out, int64_t out_layer_stride, int64_t out_row_stride,
                                         int32_t vector_ok, void* stream) {
  using namespace hla;
  HLA_REQUIRE(num_layers >= 1 && num_layers <= 65535 && length >= 0, HLA_S6_EINVAL,
              "gather_packed_rows: bad layer count or length");
  HLA_REQUIRE(main_width >= 1 && l1_width >= 1 && main_block_size >= 1 && l1_block_size >= 1, HLA_S6_EINVAL,
              "gather_packed_rows: bad widths or block sizes");
  HLA_REQUIRE(main_row_stride >= 2 * main_width && l1_row_stride >= 2 * l1_width &&
                  out_row_stride >= 2 * (main_width + l1_width) && out_layer_stride >= (int64_t)length * out_row_stride,
              HLA_S6_EINVAL, "gather_packed_rows: rows overlap (strides smaller than the row widths)");
  if (length == 0) return HLA_S6_OK;
  HLA_REQUIRE(cache_addrs && main_blocks && l1_blocks && out, HLA_S6_EINVAL, "gather_packed_rows: null pointer");
  PackParams p = {};
  p.addrs = cache_addrs;
  p.layers = num_layers;
  p.length = length;
  p.page_stride[0] = main_page_stride;
  p.page_stride[1] = l1_page_stride;
  p.row_stride[0] = main_row_stride;
  p.row_stride[1] = l1_row_stride;
  p.num_blocks[0] = main_num_blocks;
  p.num_blocks[1] = l1_num_blocks;
  p.width2[0] = 2 * main_width;
  p.width2[1] = 2 * l1_width;
  p.blocks[0] = main_blocks;
  p.blocks[1] = l1_blocks;
  p.block_size[0] = main_block_size;
  p.block_size[1] = l1_block_size;
  p.out = static_cast<uint16_t*>(out);
  p.out_layer_stride = out_layer_stride;
  p.out_row_stride = out_row_stride;
  const bool vec = vector_ok && (2 * main_width) % 8 == 0 && (2 * l1_width) % 8 == 0 && main_page_stride % 8 == 0 &&
                   main_row_stride % 8 == 0 && l1_page_stride % 8 == 0 && l1_row_stride % 8 == 0 &&
                   out_layer_stride % 8 == 0 && out_row_stride % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
  const dim3 grid((unsigned)((length + 3) / 4), (unsigned)num_layers);
  if (vec)
    hipLaunchKernelGGL(pack_rows_kernel<true>, grid, dim3(256), 0, as_stream(stream), p);
  else
    hipLaunchKernelGGL(pack_rows_kernel<false>, grid, dim3(256), 0, as_stream(stream), p);
  return check_launch("gather_packed_rows");
}
