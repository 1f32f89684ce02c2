// Building blocks shared by the MFMA attention kernels (prefill and the
// grouped-query decode): element types and their MFMAs, the swizzled LDS
// layout of K and V tiles, copies from global memory straight into LDS, the
// transposing V^T read of gfx950, and the 4-lane row reductions.
//
// MFMA operand layouts (wave64, lane l, c16 = l % 16, g4 = l / 16):
//   16x16x32: A[m][k] m = c16, k = 8 g4 + j;  B[k][n] n = c16, k = 8 g4 + j
//   16x16x16: A[m][k] m = c16, k = 4 g4 + j;  B[k][n] n = c16, k = 4 g4 + j
//   both:     C[m][n] n = c16, m = 4 g4 + i
#pragma once

#include "nkv_common.h"

namespace nkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// The element type: bf16 (kHalf false) or fp16 (kHalf true), with its 8-
// and 4-wide vectors and the matching MFMAs (fp32 accumulation).
template <bool kHalf>
struct Elem {
  typedef __bf16 T;
  typedef bf16x8 X8;
  typedef bf16x4 X4;
  static __device__ __forceinline__ f32x4 mfma(X8 a, X8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(X4 a, X4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                     __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
  }
};
template <>
struct Elem<true> {
  typedef _Float16 T;
  typedef f16x8 X8;
  typedef f16x4 X4;
  static __device__ __forceinline__ f32x4 mfma(X8 a, X8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(X4 a, X4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
};

// K and V tiles in LDS are [key][16-byte chunk] (one 256-byte head row per
// key), the chunks of key r swizzled so that the MFMA operand reads are
// conflict-free:
//   K: chunk c at c ^ (r % 16)    (ds_read_b128: 16 keys at one chunk)
//   V: chunk c at c ^ 2 (r % 8)   (ds_read_b64_tr_b16: 16 keys x 32 bytes)
__device__ __forceinline__ int k_index(int key, int chunk) {
  return key * 16 + (chunk ^ (key & 15));
}
__device__ __forceinline__ int v_index(int key, int chunk) {
  return key * 16 + (chunk ^ ((key & 7) << 1));
}

// Max / sum over the 4 lanes l, l ^ 16, l ^ 32, l ^ 48 (the lanes of one
// column of an MFMA result), with the cross-row swaps of gfx950 (no LDS
// traffic).
__device__ __forceinline__ float row4_max(float x) {
  auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float row4_sum(float x) {
  auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// One wavefront copies 16 bytes per lane from global memory straight into
// LDS: lane l's bytes land at lds_dst + 16 l (global_load_lds_dwordx4, LDS
// base in M0).  Written as asm so that the compiler, which cannot tell which
// LDS buffer such a copy writes, does not make every later LDS access wait
// for it: a kernel waits for its copies itself (s_waitcnt on the vector
// memory counter, which these copies count in, plus a barrier when other
// wavefronts read the buffer) before it reads the buffer they fill.
// M0 is a reserved register, so clang warns that a clobber of it may not be
// preserved; in the kernels built from this file every M0 access is the
// s_mov_b32 of these copies (no compiler value lives in M0 across them).
// LDS byte address of a __shared__ array (a constant once inlined).
__device__ __forceinline__ uint32_t lds_address(const u32x4* array) {
  typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_u32x4*)array));
}
// kStream: data read once (the nt cache policy, as nontemporal loads use).
// Source as a 64-bit per-lane address; lds_dst is wave-uniform.
template <bool kStream = false>
__device__ __forceinline__ void lds_copy16(const uint8_t* src, uint32_t lds_dst) {
  if constexpr (kStream) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :
                 : "v"(src), "s"(lds_dst)
                 : "m0", "memory");
  } else {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(lds_dst)
                 : "m0", "memory");
  }
}
// Source as a wave-uniform base (SGPRs) plus a per-lane 32-bit byte offset.
template <bool kStream = false>
__device__ __forceinline__ void lds_copy16(const uint8_t* base, uint32_t offset, uint32_t lds_dst) {
  if constexpr (kStream) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                 :
                 : "v"(offset), "s"(base), "s"(lds_dst)
                 : "m0", "memory");
  } else {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(offset), "s"(base), "s"(lds_dst)
                 : "m0", "memory");
  }
}

// Four consecutive elements of V^T for the PV product: lane 16 G + 4 j + q
// supplies the address of V[key][dim4 .. +4] and receives, as lane 16 G + i,
// V[key of lane 16 G + 4 j'][dim of lane 16 G + i] for j' = 0..3 (the
// gfx950 transposing LDS read).
__device__ __forceinline__ u32x2 v_tr_read(const u32x4* v_tile, int key, int dim4) {
  const int byte = (v_index(key, dim4 >> 3) << 4) + ((dim4 & 7) << 1);
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) char lds_char;
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  lds_v4i16* p = (lds_v4i16*)((lds_char*)(v_tile) + byte);  // generic -> LDS
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(p));
}

}  // namespace
}  // namespace nkv
