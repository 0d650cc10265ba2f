// Shared device helpers for the S6 latent-attention kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hla_s6.h"

namespace hla {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---- bf16 <-> f32 (bit patterns in uint16_t), round to nearest even -------------------------------
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// Conversions run on gfx950's v_cvt_pk_bf16_f32 (round to nearest even, denormals kept under the default IEEE mode).
// Its results equal the bit arithmetic u + 0x7fff + ((u >> 16) & 1) >> 16 with NaN -> (u >> 16) | 0x40 (a quiet NaN
// keeping the payload's top bits) on every value checked: the specials (NaN payloads, infinities, denormals, ties)
// and a million random bit patterns, one instruction for two values instead of about six per value.

// Pack two fp32 values into one dword of two bf16 (lo = a, hi = b).
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float float2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2_t){a, b}, bf16x2_t));
}

__device__ __forceinline__ uint16_t f2bf(float f) { return (uint16_t)(pack2(f, 0.f) & 0xffffu); }

// Round an fp32 value to the nearest bf16 value (result kept in fp32).
__device__ __forceinline__ float rbf(float f) { return __uint_as_float(pack2(f, 0.f) << 16); }

// The same conversion under its former name (softmax probabilities).
__device__ __forceinline__ uint32_t pack2_hw(float a, float b) { return pack2(a, b); }

__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// 16-byte global load / store helpers.
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// The 8 bf16 of two ds_read_b64_tr_b16 results as one 16-byte MFMA operand (lo first; a pure register view).
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x4 join_tr(short4v lo, short4v hi) {
  const u32x2 a = __builtin_bit_cast(u32x2, lo), b = __builtin_bit_cast(u32x2, hi);
  return u32x4{a[0], a[1], b[0], b[1]};
}

// ---- MFMA wrappers ----------------------------------------------------------------------------------
// 16x16x32 bf16: lane l supplies A[l%16][8*(l/16) .. +8] and B[8*(l/16) .. +8][l%16];
// D: lane l holds D[4*(l/16) + r][l%16], r = 0..3.
__device__ __forceinline__ floatx4 mfma16x16x32(u32x4 a, u32x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}
// 32x32x16 bf16: lane l supplies A[l%32][8*(l/32) .. +8] and B[8*(l/32) .. +8][l%32]; D[32][32] comes back as
// d[4j + i] = D[8j + 4*(l/32) + i][l%32], j, i < 4.
typedef float floatx16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ floatx16 mfma32x32x16(u32x4 a, u32x4 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}
// 16x16x16 bf16: lane l supplies A[l%16][4*(l/16) .. +4] and B[4*(l/16) .. +4][l%16]; D as above.
__device__ __forceinline__ floatx4 mfma16x16x16(short4v a, short4v b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Reductions across lanes l, l^16, l^32, l^48 (every lane of the four gets the same value). v_permlane16_swap with
// both operands v leaves (row 0, row 0, row 2, row 2) in one result and (row 1, row 1, row 3, row 3) in the other,
// so combining the two pairs each lane with lane l^16; v_permlane32_swap does the same for l^32. VALU only, no LDS
// round trip; the additions are the ones of the shuffle form, (v_l + v_l^16) + (v_l^32 + v_l^48).
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float wave_max16x4(float v) { return xor32_max(xor16_max(v)); }

// Maxima of values that are never NaN, without the quieting the compiler adds around fmaxf for operands it cannot
// prove canonical (two extra VALU operations per maximum).
__device__ __forceinline__ float max_nn(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max3_nn(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// wave_max16x4 for values that are never NaN
__device__ __forceinline__ float wave_max16x4_nn(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = max_nn(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max_nn(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_sum16x4(float v) { return xor32_sum(xor16_sum(v)); }


// ---- direct global -> LDS copies and the waits that go with them -----------------------------------------------
// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int waitcnt_imm(int vm, int lgkm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | ((lgkm & 15) << 8); }

// One direct global -> LDS copy of 16 bytes per lane: lane i reads 16 bytes at row + voff (row wave-uniform, voff
// the lane's byte offset) and writes them to LDS address lds + 16 i (lds wave-uniform). Issued as inline assembly
// so that the compiler neither waits for it before unrelated LDS reads (it cannot tell which tile buffer a copy
// writes) nor counts it: the caller waits for it with an explicit s_waitcnt.
__device__ __forceinline__ void copy16_to_lds(const void* row, uint32_t voff, const void* lds) {
  const uint32_t dst = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds;
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(dst), "v"(voff), "s"(row)
               : "memory", "m0");
}

// The same for callers whose LDS address the compiler may hold in a VGPR (a uniform value): it goes through
// readfirstlane into the SGPR the copy needs.
__device__ __forceinline__ void copy16_to_lds_rfl(const void* row, uint32_t voff, const void* lds) {
  const uint32_t dst =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(dst), "v"(voff), "s"(row)
               : "memory", "m0");
}

// The same with a per-lane source address (64-bit, in VGPRs).
__device__ __forceinline__ void copy16_to_lds_v(const void* src, const void* lds) {
  const uint32_t dst = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds;
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(dst), "v"(src) : "memory", "m0");
}

// 4 bytes per lane from a per-lane source address to LDS address lds + 4 i (a gather of scattered words).
__device__ __forceinline__ void copy4_to_lds_v(const void* src, const void* lds) {
  const uint32_t dst = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds;
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(dst), "v"(src) : "memory", "m0");
}

__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// A workgroup barrier that waits for nothing by itself: the caller has already waited for what other waves read
// after it. The empty asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void plain_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace hla

// ---- host-side error plumbing (api.hip) ----------------------------------------------------------
namespace hla {
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
int khop_forward_mq(const void* q, int64_t q_st, int64_t q_sh, const void* k, const void* v, int64_t k_sn, int B,
                    int Lq, int N, int width, const uint8_t* mask, int64_t mask_sb, int64_t mask_st,
                    const int32_t* bound, float scale, void* z, int64_t z_st, int64_t z_sh, float* lse,
                    hipStream_t stream);  // history.hip
}  // namespace hla

#define HLA_REQUIRE(cond, code, ...) \
  do {                               \
    if (!(cond)) return ::hla::fail((code), __VA_ARGS__); \
  } while (0)
