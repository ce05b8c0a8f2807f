// Router weight on the fc2 input: the arithmetic of the reference's non-EP
// fused MoE (TritonFusedMoeExpertFunction and
// MergedFc1TritonFusedMoeExpertFunction, veomni/ops/kernels/moe/group_gemm.py:
// 269-276, :365-406, :494-499, :577-592), which multiplies each permuted row's
// SwiGLU output by its router weight before fc2 and sums the top-k rows of a
// token unweighted afterwards.  The EP path applies the weight in the combine
// instead (routing.hip); the two agree in exact arithmetic and differ in bf16
// rounding.
//
//   forward   act_w[r] = bf16(act[r] * row_w[r])
//   backward  dact[r]  = bf16(d_act_w[r] * row_w[r])
//             dw_row[r] = bf16( sum_j fp32( bf16(act[r,j] * d_act_w[r,j]) ) )
//             dG1[r]   = SwiGLU backward of dact (swiglu_bwd8's rounding points)

#include "common.h"

namespace {

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// out[r, :] = bf16(act[r, :] * row_w[r]).  VEC: one thread per 16-byte chunk
// (N a multiple of 8), grid-stride; else one thread per element.
template <class E, bool VEC>
__global__ __launch_bounds__(256) void weight_rows_kernel(const bf16_t* __restrict__ act,
                                                          const bf16_t* __restrict__ row_w, int64_t R, int64_t N,
                                                          bf16_t* __restrict__ out) {
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  if constexpr (VEC) {
    const int64_t n8 = N / 8;
    const int64_t total = R * n8;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += step) {
      const float w = E::to_f32(row_w[e / n8]);
      float a[8];
      unpack8e<E>(ld_stream(reinterpret_cast<const uint4*>(act) + e), a);
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] *= w;
      reinterpret_cast<uint4*>(out)[e] = pack8e<E>(a);
    }
  } else {
    const int64_t total = R * N;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += step)
      out[e] = (bf16_t)E::from_f32(E::to_f32(act[e]) * E::to_f32(row_w[e / N]));
  }
}

// Scalar form of swiglu_bwd8 (same operations and rounding points).
template <class E>
__device__ __forceinline__ void swiglu_bwd1(float dact, float g, float u, float& dgate, float& dup) {
  const float sig = sigmoid_f32(g);
  const float gs = g * sig;
  dgate = E::round(dact * u) * __builtin_fmaf(gs, 1.0f - sig, sig);
  dup = E::round(gs) * dact;
}

// One wave per row, four rows per block.  Row r reads d_act_w[r], act[r] and
// gu[r] (gate | up), writes dG1[r] (d_gate | d_up) and the router-weight
// gradient dw[row_src[r]] (not written when row_src[r] lies outside [0, A)).
// The row sum: each lane sums its chunks in order (8 products per chunk, in
// column order), then the wave's lanes are summed by a butterfly.
template <class E, bool VEC>
__global__ __launch_bounds__(256) void swiglu_bwd_weighted_kernel(
    const bf16_t* __restrict__ daw, const bf16_t* __restrict__ gu, const bf16_t* __restrict__ act,
    const bf16_t* __restrict__ row_w, const int32_t* __restrict__ row_src, int64_t R, int64_t I, int64_t A,
    bf16_t* __restrict__ dg1, bf16_t* __restrict__ dw) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (r >= R) return;
  const float w = E::to_f32(row_w[r]);
  const bf16_t* d_row = daw + r * I;
  const bf16_t* a_row = act + r * I;
  const bf16_t* g_row = gu + r * 2 * I;
  bf16_t* o_row = dg1 + r * 2 * I;
  float part = 0.f;
  if constexpr (VEC) {
    const int64_t n8 = I / 8;
    for (int64_t i = lane; i < n8; i += 64) {
      float d[8], a[8], g[8], u[8], dact[8], dgate[8], dup[8];
      unpack8e<E>(ld_stream(reinterpret_cast<const uint4*>(d_row) + i), d);
      unpack8e<E>(ld_stream(reinterpret_cast<const uint4*>(a_row) + i), a);
      unpack8e<E>(ld_stream(reinterpret_cast<const uint4*>(g_row) + i), g);
      unpack8e<E>(ld_stream(reinterpret_cast<const uint4*>(g_row + I) + i), u);
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        dact[j] = d[j] * w;
        dact[j + 1] = d[j + 1] * w;
        E::round2(dact[j], dact[j + 1]);
        float p0 = a[j] * d[j], p1 = a[j + 1] * d[j + 1];
        E::round2(p0, p1);
        s += p0;
        s += p1;
      }
      part += s;
      swiglu_bwd8<E>(dact, g, u, dgate, dup);
      reinterpret_cast<uint4*>(o_row)[i] = pack8e<E>(dgate);
      reinterpret_cast<uint4*>(o_row + I)[i] = pack8e<E>(dup);
    }
  } else {
    for (int64_t j = lane; j < I; j += 64) {
      const float d = E::to_f32(d_row[j]);
      const float dact = E::round(d * w);
      part += E::round(E::to_f32(a_row[j]) * d);
      float dgate, dup;
      swiglu_bwd1<E>(dact, E::to_f32(g_row[j]), E::to_f32(g_row[I + j]), dgate, dup);
      o_row[j] = (bf16_t)E::from_f32(dgate);
      o_row[I + j] = (bf16_t)E::from_f32(dup);
    }
  }
  part = wave_sum(part);
  if (lane == 0 && dw != nullptr) {
    const int64_t k = row_src[r];
    if (k >= 0 && k < A) dw[k] = (bf16_t)E::from_f32(part);
  }
}


template <class E>
int weight_rows_t(const void* act, const void* row_w, int64_t R, int64_t N, void* out, pmx_stream_t stream) {
  if (R < 0 || N < 0) return PMX_ERR_ARG;
  if (R == 0 || N == 0) return PMX_OK;
  if (!act || !row_w || !out) return PMX_ERR_ARG;
  if (R > INT64_MAX / N) return PMX_ERR_SHAPE;
  const bool vec = N % 8 == 0 && aligned16(act) && aligned16(out);
  const int64_t work = vec ? R * (N / 8) : R * N;
  const int64_t blocks = (work + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 16384 ? blocks : 16384);
  if (vec)
    weight_rows_kernel<E, true><<<grid, 256, 0, stream>>>((const bf16_t*)act, (const bf16_t*)row_w, R, N,
                                                          (bf16_t*)out);
  else
    weight_rows_kernel<E, false><<<grid, 256, 0, stream>>>((const bf16_t*)act, (const bf16_t*)row_w, R, N,
                                                           (bf16_t*)out);
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}

template <class E>
int swiglu_bwd_weighted_t(const void* d_act_w, const void* gu, const void* act, const void* row_w,
                            const int32_t* row_src, int64_t R, int64_t I, int64_t A, void* dG1, void* dw,
                            pmx_stream_t stream) {
  if (R < 0 || I < 0 || A < 0) return PMX_ERR_ARG;
  if ((dw == nullptr) != (row_src == nullptr)) return PMX_ERR_ARG;
  if (R == 0) return PMX_OK;
  if (!row_w || (I > 0 && (!d_act_w || !gu || !act || !dG1))) return PMX_ERR_ARG;
  if ((R + 3) / 4 > (int64_t)INT32_MAX || (I > 0 && R > INT64_MAX / (2 * I))) return PMX_ERR_SHAPE;
  const bool vec = I % 8 == 0 && aligned16(d_act_w) && aligned16(gu) && aligned16(act) && aligned16(dG1);
  const unsigned grid = (unsigned)((R + 3) / 4);
  if (vec)
    swiglu_bwd_weighted_kernel<E, true><<<grid, 256, 0, stream>>>(
        (const bf16_t*)d_act_w, (const bf16_t*)gu, (const bf16_t*)act, (const bf16_t*)row_w, row_src, R, I, A,
        (bf16_t*)dG1, (bf16_t*)dw);
  else
    swiglu_bwd_weighted_kernel<E, false><<<grid, 256, 0, stream>>>(
        (const bf16_t*)d_act_w, (const bf16_t*)gu, (const bf16_t*)act, (const bf16_t*)row_w, row_src, R, I, A,
        (bf16_t*)dG1, (bf16_t*)dw);
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}

}  // namespace

extern "C" {

int pmx_weight_rows(const void* act, const void* row_w, int64_t R, int64_t N, void* out, pmx_stream_t stream) {
  return weight_rows_t<EltBF16>(act, row_w, R, N, out, stream);
}

int pmx_weight_rows_f16(const void* act, const void* row_w, int64_t R, int64_t N, void* out, pmx_stream_t stream) {
  return weight_rows_t<EltF16>(act, row_w, R, N, out, stream);
}


int pmx_swiglu_bwd_weighted(const void* d_act_w, const void* gu, const void* act, const void* row_w,
                            const int32_t* row_src, int64_t R, int64_t I, int64_t A, void* dG1, void* dw,
                            pmx_stream_t stream) {
  return swiglu_bwd_weighted_t<EltBF16>(d_act_w, gu, act, row_w, row_src, R, I, A, dG1, dw, stream);
}

int pmx_swiglu_bwd_weighted_f16(const void* d_act_w, const void* gu, const void* act, const void* row_w,
                                const int32_t* row_src, int64_t R, int64_t I, int64_t A, void* dG1, void* dw,
                                pmx_stream_t stream) {
  return swiglu_bwd_weighted_t<EltF16>(d_act_w, gu, act, row_w, row_src, R, I, A, dG1, dw, stream);
}


}  // extern "C"
