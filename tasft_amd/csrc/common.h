// Shared device/host helpers for the gfx950 block-sparse attention kernels.
//
// Everything here is CDNA4-specific: wave64, bf16/fp16 MFMA (v_mfma_f32_32x32x16_{bf16,f16}),
// and the 64-bank LDS of gfx950. No CUDA compatibility layer is used.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace tasft {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

#define TASFT_LDS __attribute__((address_space(3)))

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// Status codes returned by every extern "C" entry point.
enum Status : int {
  kOk = 0,
  kErrInvalidArgument = -1,
  kErrUnsupported = -2,
  kErrLaunch = -3,
  kErrWorkspace = -4,
};

// Thread-local last-error message (defined in capi.cpp).
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// True if none of the n element strides is negative: the kernels index forward from each
// tensor's base pointer.
inline bool strides_nonneg(const int64_t* s, int n) {
  for (int i = 0; i < n; ++i)
    if (s[i] < 0) return false;
  return true;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Unpack 8 bf16 (as uint4) to 8 floats.
__device__ __forceinline__ void unpack_bf16x8(const u32x4_t& v, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(v[i] << 16);
    out[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even fp32 -> bf16 of two values packed in one dword
// (one v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ f32x16_t mfma_32x32x16_bf16(const bf16x8_t& a, const bf16x8_t& b,
                                                        const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t& v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// Element type of the 16-bit tensors (Q, K, V, out). The kernels move them as raw 16-bit
// words; only the MFMA that multiplies them, the fp32 -> 16-bit rounding (P before the PV
// product, the output) and the 16-bit -> fp32 unpack depend on it. Values match
// TASFT_DTYPE_BF16 / TASFT_DTYPE_F16 of the C ABI.
enum DType : int { kBf16 = 0, kF16 = 1 };

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// v_mfma_f32_32x32x16_{bf16,f16}: 8 elements per lane of A and B as raw words.
template <int DT>
__device__ __forceinline__ f32x16_t mfma16(const u32x4_t& a, const u32x4_t& b, const f32x16_t& c) {
  if constexpr (DT == kF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Round-to-nearest-even fp32 -> 16-bit of two values packed in one dword (lo in bits 0-15).
template <int DT>
__device__ __forceinline__ uint32_t pack16x2(float lo, float hi) {
  if constexpr (DT == kF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, f16x2_t));
  else
    return pack_bf16x2(lo, hi);
}

// Unpack 8 16-bit values (as uint4) to 8 floats.
template <int DT>
__device__ __forceinline__ void unpack16x8(const u32x4_t& v, float* out) {
  if constexpr (DT == kF16) {
    const f16x8_t h = __builtin_bit_cast(f16x8_t, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = (float)h[i];
  } else {
    unpack_bf16x8(v, out);
  }
}

// Round-to-nearest-even fp32 -> one 16-bit value.
template <int DT>
__device__ __forceinline__ uint16_t f32_to16(float x) {
  if constexpr (DT == kF16)
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  else
    return __builtin_bit_cast(uint16_t, (__bf16)x);
}

// One 16-bit value (low bits of `bits16`) to fp32.
template <int DT>
__device__ __forceinline__ float bits16_to_f32(uint32_t bits16) {
  if constexpr (DT == kF16)
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  else
    return bf16_bits_to_f32(bits16);
}

// gfx950 transposing LDS read (ds_read_b64_tr_b16). Within each group of 16 lanes,
// lane t receives element t%4 of the 8-byte chunks addressed by lanes t/4, t/4+4,
// t/4+8 and t/4+12 of its group. If source lane s addresses row R0 + s/4, columns
// C0 + 4*(s%4) .. +3 of a row-major 16-bit matrix, lane t receives rows R0..R0+3 of
// column C0 + t: a 4x16 tile read transposed.
__device__ __forceinline__ u32x2_t ds_read_tr16_b64(const void* lds_byte_addr) {
  const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TASFT_LDS i16x4_t*)lds_byte_addr);
  return __builtin_bit_cast(u32x2_t, v);
}

// Exchange a value with the lane 32 positions away (lane l <-> lane l^32).
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// max / sum of a value over the lane pair (l, l^32) with v_permlane32_swap (gfx950):
// swapping the upper half of one copy with the lower half of another leaves the pair's
// two values in the two results, in the same order on both lanes.
__device__ __forceinline__ float pair_max32(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum32(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// One DPP move (row/quad permutation of lanes) of a float.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Max over all 64 lanes without LDS traffic: a butterfly of quad permutes (xor 1, xor 2),
// half-row and row mirrors (8- and 16-lane groups), then the 16- and 32-lane swaps.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
  const uint32_t u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  return pair_max32(v);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Map a linear workgroup index onto (group, member) so that every member of a
// group lands on the same XCD. gfx950 in SPX mode dispatches workgroup i to XCD
// i % 8, so a group of `members` items sharing data (the query heads of one KV
// head) is placed on one XCD and shares that XCD's L2. Requires
// num_groups % 8 == 0; otherwise the identity mapping is used.
__device__ __forceinline__ void xcd_group_map(int64_t idx, int64_t num_groups, int members,
                                              int64_t* group, int* member) {
  if ((num_groups & 7) == 0) {
    const int64_t xcd = idx & 7;
    const int64_t j = idx >> 3;
    *group = xcd + 8 * (j / members);
    *member = (int)(j % members);
  } else {
    *group = idx / members;
    *member = (int)(idx % members);
  }
}

}  // namespace tasft
