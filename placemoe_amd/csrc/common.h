// Shared helpers for the gfx950 kernels of the PlaceMoE expert-layer path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/placemoe_amd.h"

#define PMX_WAVE 64

typedef uint16_t bf16_t;  // bf16 bit pattern in memory

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// bf16 -> fp32 is exact: the bf16 bits are the top half of the fp32 word.
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16, round to nearest even; NaN stays NaN.  gfx950 converts in
// hardware (v_cvt_pk_bf16_f32); checked on the device against the integer
// round-to-nearest-even formula over all 2^32 fp32 patterns: identical for
// every non-NaN input, NaN for every NaN input.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Two fp32 -> a bf16 pair (a in the low half) in one v_cvt_pk_bf16_f32, with
// the same rounding as f32_to_bf16.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// round_bf16 of two values through one conversion.
__device__ __forceinline__ void round2_bf16(float& a, float& b) {
  const uint32_t p = pack2(a, b);
  a = __uint_as_float(p << 16);
  b = __uint_as_float(p & 0xffff0000u);
}

// Unpack / pack 8 bf16 held in a uint4 (element 2j in the low half of word j).
__device__ __forceinline__ void unpack8(const uint4 v, float* f) {
  f[0] = __uint_as_float(v.x << 16); f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16); f[3] = __uint_as_float(v.y & 0xffff0000u);
  f[4] = __uint_as_float(v.z << 16); f[5] = __uint_as_float(v.z & 0xffff0000u);
  f[6] = __uint_as_float(v.w << 16); f[7] = __uint_as_float(v.w & 0xffff0000u);
}

__device__ __forceinline__ uint4 pack8(const float* f) {
  return make_uint4(pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7]));
}

// 16-bit element types of the float path (bf16 and fp16).  Row copies and
// the GEMMs' operand paths move 16-bit patterns without reading them; an
// element type fixes only the conversions to and from fp32 (round to nearest
// even, as torch's .to(dtype)) and, in the GEMM, the MFMA that multiplies
// it.  to_f32 reads the low 16 bits of its argument.
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
struct EltBF16 {
  static constexpr int kCode = 0;
  __device__ static __forceinline__ float to_f32(uint32_t b) { return bf16_to_f32(b & 0xffffu); }
  __device__ static __forceinline__ uint32_t pack2(float a, float b) { return ::pack2(a, b); }
  __device__ static __forceinline__ uint32_t from_f32(float f) { return f32_to_bf16(f); }
  __device__ static __forceinline__ float round(float f) { return round_bf16(f); }
  __device__ static __forceinline__ void round2(float& a, float& b) { round2_bf16(a, b); }
  __device__ static __forceinline__ void unpack2(uint32_t w, float& a, float& b) {
    a = __uint_as_float(w << 16);
    b = __uint_as_float(w & 0xffff0000u);
  }
};
// fp16: gfx950 converts a pair in one v_cvt_pk_f16_f32 (round to nearest
// even, overflow to inf) and widens with v_cvt_f32_f16 (exact).
struct EltF16 {
  static constexpr int kCode = 2;
  __device__ static __forceinline__ float to_f32(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xffffu));
  }
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
  }
  __device__ static __forceinline__ uint32_t from_f32(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
  }
  __device__ static __forceinline__ float round(float f) { return (float)(_Float16)f; }
  __device__ static __forceinline__ void round2(float& a, float& b) {
    const f16x2_t h = __builtin_bit_cast(f16x2_t, pack2(a, b));
    a = (float)h[0];
    b = (float)h[1];
  }
  __device__ static __forceinline__ void unpack2(uint32_t w, float& a, float& b) {
    const f16x2_t h = __builtin_bit_cast(f16x2_t, w);
    a = (float)h[0];
    b = (float)h[1];
  }
};

// unpack8 / pack8 of either element type (element 2j in the low half of word j).
template <class E>
__device__ __forceinline__ void unpack8e(const uint4 v, float* f) {
  E::unpack2(v.x, f[0], f[1]);
  E::unpack2(v.y, f[2], f[3]);
  E::unpack2(v.z, f[4], f[5]);
  E::unpack2(v.w, f[6], f[7]);
}
template <class E>
__device__ __forceinline__ uint4 pack8e(const float* f) {
  return make_uint4(E::pack2(f[0], f[1]), E::pack2(f[2], f[3]), E::pack2(f[4], f[5]), E::pack2(f[6], f[7]));
}

// Dispatch on the element code a C-ABI entry point passes (0 bf16, 2 fp16):
// LAUNCH(E) with E the element type.
#define PMX_DISPATCH_ELT(code, LAUNCH) \
  do {                                 \
    if ((code) == EltF16::kCode) {     \
      LAUNCH(EltF16);                  \
    } else {                           \
      LAUNCH(EltBF16);                 \
    }                                  \
  } while (0)

// 16-byte streaming (non-temporal) global load and store, for row data that
// a kernel touches exactly once.  Measured on the row-movement kernels inside
// the layer: streaming loads are 5-20% faster than plain loads; streaming
// stores are faster only where each token writes a single row (top-1), and
// slower where it writes K > 1 rows, so the kernels choose per call.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_stream(void* p, const uint4 v) {
  __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(p));
}
template <bool STREAM>
__device__ __forceinline__ void st_row(void* p, const uint4 v) {
  if constexpr (STREAM) st_stream(p, v);
  else *reinterpret_cast<uint4*>(p) = v;
}

// sigmoid(x) = 1 / (1 + exp(-x)) with the hardware exponential (__expf) and
// reciprocal (v_rcp_f32, 1 ulp) instead of an IEEE division, and silu(x) =
// x * sigmoid(x): a few ulp of fp32 from the correctly rounded quotient, which
// the kernels' outputs then round to bf16.  The divisions were the bulk of the
// GEMM epilogues' VALU work, which holds the matrix cores idle.
__device__ __forceinline__ float sigmoid_f32(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float silu_f32(float x) { return x * sigmoid_f32(x); }

// SwiGLU backward of 8 columns, with the reference's rounding points
// (aten silu_backward and the products around it in
// EPMergedFc1GroupGemm.backward, veomni/distributed/moe/moe_layer.py:453-482,
// :479): dact is the bf16 dgrad output,
//   s = bf16(silu(g)), d_silu = bf16(dact * u), sig = sigmoid(g)
//   dgate = d_silu * sig * (1 + g * (1 - sig)),  dup = s * dact,
// with sig * (1 + g * (1 - sig)) evaluated as sig + silu(g) * (1 - sig) in
// one fma (fp32 rounding differs from aten's order by a few ulp).  E: the
// element type whose rounding the bf16 points above take (fp16 for fp16).
template <class E = EltBF16>
__device__ __forceinline__ void swiglu_bwd8(const float* dact, const float* g, const float* u, float* dgate,
                                            float* dup) {
#pragma unroll
  for (int q = 0; q < 8; q += 2) {
    const float sig0 = sigmoid_f32(g[q]), sig1 = sigmoid_f32(g[q + 1]);
    const float gs0 = g[q] * sig0, gs1 = g[q + 1] * sig1;
    float s0 = gs0, s1 = gs1;
    float d0 = dact[q] * u[q], d1 = dact[q + 1] * u[q + 1];
    E::round2(s0, s1);
    E::round2(d0, d1);
    dgate[q] = d0 * __builtin_fmaf(gs0, 1.0f - sig0, sig0);
    dgate[q + 1] = d1 * __builtin_fmaf(gs1, 1.0f - sig1, sig1);
    dup[q] = s0 * dact[q];
    dup[q + 1] = s1 * dact[q + 1];
  }
}

// Wave-wide sum (64 lanes) with cross-lane shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, PMX_WAVE);
  return v;
}

static inline int pmx_status(hipError_t e) { return e == hipSuccess ? PMX_OK : PMX_ERR_HIP; }

// The routing path's stable counting sort (routing.hip), shared with the
// expert-parallel payload builder (payload.hip); not part of the C ABI.
__attribute__((visibility("hidden"))) int pmx_route_launch(
    const int64_t* sel, const int64_t* M, const int64_t* src, int32_t src_const, int32_t S, int32_t E, int64_t A,
    int32_t K, int32_t C, int32_t* phys, int32_t* counts, int32_t* offsets, int32_t* pos, void* workspace,
    size_t workspace_bytes, hipStream_t stream);
__attribute__((visibility("hidden"))) size_t pmx_route_ws_bytes(int64_t A, int32_t C);

#define PMX_LAUNCH_CHECK()                         \
  do {                                             \
    hipError_t _e = hipGetLastError();             \
    if (_e != hipSuccess) return PMX_ERR_HIP;      \
  } while (0)
