// Shared device helpers for the Motif Chord HIP kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace motif {

constexpr float kLog2e = 1.4426950408889634f;

typedef uint16_t bf16_t;  // raw bfloat16 storage

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

__device__ __forceinline__ float bf16_to_f32(bf16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN): the gfx950 conversion
// instruction (v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
};
template <> struct Elem<bf16_t> {
  __device__ __forceinline__ static float load(const bf16_t* p) { return bf16_to_f32(*p); }
  __device__ __forceinline__ static void store(bf16_t* p, float v) { *p = f32_to_bf16(v); }
};

typedef _Float16 f16_t;  // IEEE half
template <> struct Elem<f16_t> {
  __device__ __forceinline__ static float load(const f16_t* p) { return static_cast<float>(*p); }
  __device__ __forceinline__ static void store(f16_t* p, float v) { *p = static_cast<f16_t>(v); }
};

template <typename T> __device__ __forceinline__ float ld(const T* p) { return Elem<T>::load(p); }
template <typename T> __device__ __forceinline__ void st(T* p, float v) { Elem<T>::store(p, v); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// exp(x) through the hardware exp2 with the argument pre-scaled.
__device__ __forceinline__ float exp_f(float x) { return exp2f(x * kLog2e); }

// 1 / x as one v_rcp_f32 (1 ulp).
__device__ __forceinline__ float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }

// x * sigmoid(x) with the single-instruction exp and reciprocal.
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// exp(x) as one v_exp_f32 (1 ulp, no denormal range handling: results below
// 2^-126 may flush to zero) -- for decay factors e^{gamma_i - gamma_j} <= 1.
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// Raw buffer over [base, base + bytes) (uniform base and size): a load whose byte
// offset falls outside returns zeros by the hardware range check, so bounded tile
// loads need no branches (a load under a lane-varying branch is followed by a wait,
// which serialises a batch of loads).  Negative offsets wrap to large unsigned ones.
typedef __amdgpu_buffer_rsrc_t buf_t;
__device__ __forceinline__ buf_t make_buf(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_ld16(buf_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// The same load marked nontemporal (cache-policy operand 2: the `nt` bit on gfx950), for
// data a kernel streams once (KV caches, recurrent states): it is not kept in the caches
// at the expense of data that is reused.
__device__ __forceinline__ uint4 buf_ld16_nt(buf_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}
// 16 bytes per lane straight from a buffer into LDS at dst + 16 * lane (dst the same
// for the whole wave; offsets past the range write zeros); AUX is the cache policy.
typedef __attribute__((address_space(3))) void lds_void;
template <int AUX = 0>
__device__ __forceinline__ void buf_ld16_lds(buf_t r, void *dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 16, voff, soff, 0, AUX);
}
__device__ __forceinline__ uint2 buf_ld8(buf_t r, uint32_t off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
template <typename T> __device__ __forceinline__ float buf_ld(buf_t r, uint32_t elem);
template <> __device__ __forceinline__ float buf_ld<float>(buf_t r, uint32_t elem) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, elem * 4, 0, 0));
}
template <> __device__ __forceinline__ float buf_ld<bf16_t>(buf_t r, uint32_t elem) {
  return bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, elem * 2, 0, 0));
}

// x rounded to the storage type T and back (identity for float).
template <typename T> __device__ __forceinline__ float round_as(float x) { return x; }
template <> __device__ __forceinline__ float round_as<bf16_t>(float x) { return bf16_to_f32(f32_to_bf16(x)); }
template <> __device__ __forceinline__ float round_as<f16_t>(float x) { return static_cast<float>(static_cast<f16_t>(x)); }

// The GatedDelta q / k / v front end in the arithmetic of the reference layer run in the
// activation type T (motif/block/attention/gdn_attn.py:116-136, :187-191): the causal
// conv's output is rounded to T, SiLU of that value is rounded to T; F.normalize takes
// the vector norm (fp32 sum of squares) rounded to T and clamped at eps, the quotient
// rounded to T, and q's product with dk^-1/2 rounded to T (a product with 1 for k is
// exact).  The quotient is formed as y * (1 / denom), the reciprocal taken once per
// vector and refined by one Newton step: within about one fp32 ulp of the quotient, so its
// rounding to bf16 is the reference's except when the quotient falls within that ulp of a
// bf16 rounding boundary (a few elements in 10^5, one bf16 ulp each); an IEEE division
// per element costs about ten instructions.
template <typename T> __device__ __forceinline__ float gdn_conv_act(float acc) {
  return round_as<T>(silu_fast(round_as<T>(acc)));
}
// 1 / max(T(||y||), T(eps)) from the sum of squares
template <typename T> __device__ __forceinline__ float gdn_norm_inv(float sum_sq) {
  const float d = fmaxf(round_as<T>(sqrtf(sum_sq)), round_as<T>(1e-12f));
  const float r = __builtin_amdgcn_rcpf(d);
  return fmaf(r, fmaf(-d, r, 1.f), r);
}
template <typename T> __device__ __forceinline__ float gdn_normalized(float y, float inv, float scale) {
  return round_as<T>(round_as<T>(y * inv) * scale);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

}  // namespace motif
