// Replica-gradient fold on gfx950: fp32 sum of the bf16 (or fp16) gradients of every
// physical copy of a logical expert, optionally written back to the copies.
// A bandwidth kernel: each thread owns 8 consecutive elements of one expert
// and streams them from every copy with 16-byte loads.

#include "common.h"

namespace {

template <class E, bool VEC>
__global__ __launch_bounds__(256) void replica_fold_kernel(bf16_t* __restrict__ grads,
                                                           const int32_t* __restrict__ copy_offsets,
                                                           const int32_t* __restrict__ copy_slots,
                                                           const int64_t* __restrict__ slot_tokens, int32_t C,
                                                           int64_t P, float* __restrict__ out, int writeback,
                                                           int32_t* __restrict__ status) {
  const int64_t e = blockIdx.y;
  const int32_t b = copy_offsets[e], end = copy_offsets[e + 1];
  // A copy-table entry outside [0, C) is skipped in both the sum and the
  // write-back and flagged once, by the expert's first block.
  bool bad = false;
  if (VEC) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i >= P) return;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int32_t j = b; j < end; ++j) {
      const int64_t c = copy_slots[j];
      if (c < 0 || c >= C) {
        bad = true;
        continue;
      }
      if (slot_tokens != nullptr && slot_tokens[c] <= 0) continue;
      float f[8];
      unpack8e<E>(ld_stream(grads + c * P + i), f);
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] += f[q];
    }
    float4* o = reinterpret_cast<float4*>(out + e * P + i);
    o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    if (writeback) {
      const uint4 v = pack8e<E>(acc);
      for (int32_t j = b; j < end; ++j) {
        const int64_t c = copy_slots[j];
        if (c >= 0 && c < C) *reinterpret_cast<uint4*>(grads + c * P + i) = v;
      }
    }
  } else {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= P) return;
    float acc = 0.f;
    for (int32_t j = b; j < end; ++j) {
      const int64_t c = copy_slots[j];
      if (c < 0 || c >= C) {
        bad = true;
        continue;
      }
      if (slot_tokens != nullptr && slot_tokens[c] <= 0) continue;
      acc += E::to_f32(grads[c * P + i]);
    }
    out[e * P + i] = acc;
    if (writeback) {
      const bf16_t v = (bf16_t)E::from_f32(acc);
      for (int32_t j = b; j < end; ++j) {
        const int64_t c = copy_slots[j];
        if (c >= 0 && c < C) grads[c * P + i] = v;
      }
    }
  }
  if (bad && status != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *status = 1;
}


// El: the element type of the copies' gradients.
template <class El>
int replica_fold_t(void* grads, const int32_t* copy_offsets, const int32_t* copy_slots, const int64_t* slot_tokens,
                   int32_t E, int32_t C, int64_t P, float* out, int32_t writeback, int32_t* status,
                   pmx_stream_t stream) {
  if (E <= 0 || C <= 0 || P < 0 || E > 65535) return PMX_ERR_ARG;
  if (P == 0) return PMX_OK;
  if (!grads || !copy_offsets || !copy_slots || !out) return PMX_ERR_ARG;
  const bool vec = (P % 8 == 0) && ((reinterpret_cast<uintptr_t>(grads) & 15u) == 0) &&
                   ((reinterpret_cast<uintptr_t>(out) & 15u) == 0);
  const int64_t per_block = vec ? 256 * 8 : 256;
  const int64_t gx = (P + per_block - 1) / per_block;
  if (gx > 0x7fffffff) return PMX_ERR_SHAPE;
  dim3 grid((unsigned)gx, (unsigned)E);
  if (vec) {
    replica_fold_kernel<El, true><<<grid, 256, 0, stream>>>(static_cast<bf16_t*>(grads), copy_offsets, copy_slots,
                                                        slot_tokens, C, P, out, writeback, status);
  } else {
    replica_fold_kernel<El, false><<<grid, 256, 0, stream>>>(static_cast<bf16_t*>(grads), copy_offsets, copy_slots,
                                                         slot_tokens, C, P, out, writeback, status);
  }
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}

}  // namespace

extern "C" int pmx_replica_fold(void* grads, const int32_t* copy_offsets, const int32_t* copy_slots,
                                const int64_t* slot_tokens, int32_t E, int32_t C, int64_t P, float* out,
                                int32_t writeback, int32_t* status, pmx_stream_t stream) {
  return replica_fold_t<EltBF16>(grads, copy_offsets, copy_slots, slot_tokens, E, C, P, out, writeback, status,
                                stream);
}

extern "C" int pmx_replica_fold_f16(void* grads, const int32_t* copy_offsets, const int32_t* copy_slots,
                                    const int64_t* slot_tokens, int32_t E, int32_t C, int64_t P, float* out,
                                    int32_t writeback, int32_t* status, pmx_stream_t stream) {
  return replica_fold_t<EltF16>(grads, copy_offsets, copy_slots, slot_tokens, E, C, P, out, writeback, status,
                                stream);
}

