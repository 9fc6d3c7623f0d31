// hprms_device.h - device-side building blocks for gfx950 (CDNA4, wave64).
//
//   * 16-byte buffer loads/stores through a per-workgroup buffer resource, so
//     that out-of-range lanes read zeros and drop their stores in hardware
//     instead of branching (raw buffers: a lane is out of range when its
//     byte offset >= num_records).
//   * bfloat16 / binary16 pack and unpack.  Packing uses gfx950's
//     v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 (round to nearest even).
//   * wave64 sum reduction: DPP quad_perm and row mirrors inside each 16-lane
//     row, ds_swizzle across the two rows of a 32-lane half, readlane across
//     the halves.  Every lane of a group ends with the same bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hp_rms_norm_amd.h"

namespace hprms {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Word 3 of a raw (unswizzled, stride 0) buffer resource on gfx9 parts.
constexpr int kRsrcWord3 = 0x00020000;
// A byte offset past every num_records the kernels build (they stay < 2^31).
constexpr uint32_t kOOB = 0x80000000u;
// Cache-policy field of buffer instructions on gfx940+: sc0 = 1, nt
// (streaming) = 2, sc1 = 16.
constexpr int kAuxSC0 = 1;
constexpr int kAuxNT = 2;
constexpr int kAuxSC1 = 16;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}

template <int AUX>
__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
}

template <int AUX>
__device__ __forceinline__ void store16(u32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, AUX);
}

// v through an empty asm statement (no instruction): what is computed from it
// can neither move ahead of this point nor be hoisted out of a loop.  The
// kernels read their non-preloaded arguments this way after the row loads.
template <typename T>
__device__ __forceinline__ T opaque(T v) {
  asm volatile("" : "+s"(v));
  return v;
}

// ---- element formats --------------------------------------------------------
template <int DT>
struct Fmt;

// olo / ohi: the same unpacks as lo / hi, through a byte permute
// (v_perm_b32), which the compiler does not merge with lo / hi (the bench
// library's variant of the output phase, fused_vec_kernel FLAGS bit 12).
template <>
struct Fmt<HPRMS_DTYPE_BF16> {
  __device__ static __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  __device__ static __forceinline__ float olo(uint32_t w) {
    return __uint_as_float(__builtin_amdgcn_perm(0u, w, 0x01000c0cu));
  }
  __device__ static __forceinline__ float ohi(uint32_t w) {
    return __uint_as_float(__builtin_amdgcn_perm(0u, w, 0x03020c0cu));
  }
  __device__ static __forceinline__ uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  }
  __device__ static __forceinline__ float one(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
  __device__ static __forceinline__ uint16_t pack1(float a) { return (uint16_t)(pack(a, 0.0f) & 0xffffu); }
};

template <>
struct Fmt<HPRMS_DTYPE_FP16> {
  __device__ static __forceinline__ float lo(uint32_t w) {
    return (float)__builtin_bit_cast(f16x2, w)[0];
  }
  __device__ static __forceinline__ float hi(uint32_t w) {
    return (float)__builtin_bit_cast(f16x2, w)[1];
  }
  __device__ static __forceinline__ float olo(uint32_t w) {
    return (float)__builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0u, w, 0x0c0c0100u))[0];
  }
  __device__ static __forceinline__ float ohi(uint32_t w) {
    return (float)__builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0u, w, 0x0c0c0302u))[0];
  }
  __device__ static __forceinline__ uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  }
  __device__ static __forceinline__ float one(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
  __device__ static __forceinline__ uint16_t pack1(float a) { return (uint16_t)(pack(a, 0.0f) & 0xffffu); }
};

// ---- FP8 ----------------------------------------------------------------------
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Four binary32 values to four OCP e4m3fn bytes (gfx950 v_cvt_pk_fp8_f32:
// round to nearest even; callers clamp to +-448 first).  Byte i of the result
// holds value i.
__device__ __forceinline__ uint32_t pack_e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// Clamp to the e4m3fn range; NaN passes through (both compares are false).
__device__ __forceinline__ float clamp_e4m3(float v) {
  return v > 448.0f ? 448.0f : (v < -448.0f ? -448.0f : v);
}

template <int AUX>
__device__ __forceinline__ void store8(u32x2 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, AUX);
}

template <int AUX>
__device__ __forceinline__ void store4(uint32_t v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, AUX);
}

template <int AUX>
__device__ __forceinline__ void store1(uint8_t v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b8(v, r, off, 0, AUX);
}

// ---- OCP MX (E2M1 elements) ----------------------------------------------------------
// Two binary32 values to two E2M1 codes in byte SEL of w, the first value in
// the low nibble (gfx950 v_cvt_scalef32_pk_fp4_f32 with scale 1.0: round to
// nearest even, saturating at +-6; NaN gives code 7 with NaN's sign).  The
// other bytes of w are kept.
template <int SEL>
__device__ __forceinline__ uint32_t cvt_e2m1x2(uint32_t w, float a, float b) {
  return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a, b, 1.0f, SEL);
}

// ---- workgroup order ------------------------------------------------------------
// The hardware hands consecutive workgroups of a grid to the 8 XCDs in turn,
// so with work unit g = blockIdx.x XCD k always takes the units g % 8 == k.
// xcd_xor: unit g ^ ((g >> 3) & 7), so an XCD's units cycle through all 8
// residues modulo 8 in every run of 64.  xcd_runs<V>: in every block of
// 8 * 2^V units each XCD takes 2^V consecutive units (V = 3: each 8 x 8 block
// transposed).  Both permute each whole run or block of the n units; a
// trailing partial one keeps its order.
__device__ __forceinline__ int64_t xcd_xor(int64_t g, int64_t n) {
  return (g | 63) >= n ? g : g ^ ((g >> 3) & 7);
}

template <int V>
__device__ __forceinline__ int64_t xcd_runs(int64_t g, int64_t n) {
  if constexpr (V == 0) {
    return g;
  } else {
    constexpr int64_t R = int64_t(1) << V;
    if ((g | (8 * R - 1)) >= n) return g;
    return (g & ~(8 * R - 1)) | ((g & 7) << V) | ((g >> 3) & (R - 1));
  }
}

// ---- reductions ---------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}

// Sum over aligned groups of WIDTH lanes (16, 32 or 64).  Must be called with
// every lane of the wave active.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(WIDTH == 16 || WIDTH == 32 || WIDTH == 64, "group width");
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror: quads 0<->1 of each 8
  v += dpp_f32<0x140>(v);  // row_mirror: halves of each 16-lane row
  if constexpr (WIDTH >= 32) {
    // ds_swizzle bit mode: and_mask 0x1f, or_mask 0, xor_mask 0x10
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
  }
  if constexpr (WIDTH == 64) {
    v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)) +
        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  }
  return v;
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// Unsigned maximum over each aligned quad of lanes (every lane gets it).
__device__ __forceinline__ uint32_t quad_max_u32(uint32_t v) {
  v = __builtin_elementwise_max(v, dpp_u32<0xB1>(v));  // quad_perm [1,0,3,2]
  return __builtin_elementwise_max(v, dpp_u32<0x4E>(v));  // quad_perm [2,3,0,1]
}

// Unsigned maximum over aligned groups of WIDTH lanes, same lane pattern as
// group_sum.  Must be called with every lane of the wave active.
template <int WIDTH>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
  static_assert(WIDTH == 16 || WIDTH == 32 || WIDTH == 64, "group width");
  v = __builtin_elementwise_max(v, dpp_u32<0xB1>(v));
  v = __builtin_elementwise_max(v, dpp_u32<0x4E>(v));
  v = __builtin_elementwise_max(v, dpp_u32<0x141>(v));
  v = __builtin_elementwise_max(v, dpp_u32<0x140>(v));
  if constexpr (WIDTH >= 32) v = __builtin_elementwise_max(v, (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401F));
  if constexpr (WIDTH == 64)
    v = __builtin_elementwise_max((uint32_t)__builtin_amdgcn_readlane((int)v, 0),
                                  (uint32_t)__builtin_amdgcn_readlane((int)v, 32));
  return v;
}

}  // namespace hprms
