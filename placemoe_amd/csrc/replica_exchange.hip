// Per-rank halves of the cross-rank replica-gradient exchange on gfx950.
//
// A logical expert whose copies live on several EP ranks has its copy
// gradients summed across those ranks.  Each rank packs, per exchanged item
// (one logical expert x one parameter), the sum of its local copies into the
// buffer it sends to a peer; after the transfer it adds what it received to
// its own sum and writes the total into every local copy (and, on an owner
// rank, into the buffers it broadcasts back).  Both halves are one kernel: an
// item's total is
//     [sum over its local slots of grads[slot]]  +  sum over its received parts,
// accumulated in fp32 and stored in the gradient dtype, written to every
// local slot and/or to every output buffer of the item.
//
// A bandwidth kernel: blockIdx.y is the item, each thread owns 16 bytes of
// it and streams them from every source (16-byte loads where the address
// allows, element loads otherwise).

#include "common.h"

namespace {

// Element types of the exchanged gradients, by tag: EltBF16 and EltF16
// (16-bit storage) or float; S is the storage type.
template <typename T>
struct Elem;
template <class E16>
struct Elem16 {
  using S = bf16_t;
  static constexpr int kVec = 8;
  __device__ static float load(const S* p) { return E16::to_f32(*p); }
  __device__ static void store(S* p, float v) { *p = (S)E16::from_f32(v); }
  __device__ static void load_vec(const S* p, float* f) { unpack8e<E16>(ld_stream(p), f); }
  __device__ static void store_vec(S* p, const float* f) { *reinterpret_cast<uint4*>(p) = pack8e<E16>(f); }
};
template <>
struct Elem<EltBF16> : Elem16<EltBF16> {};
template <>
struct Elem<EltF16> : Elem16<EltF16> {};
template <>
struct Elem<float> {
  using S = float;
  static constexpr int kVec = 4;
  __device__ static float load(const float* p) { return *p; }
  __device__ static void store(float* p, float v) { *p = v; }
  __device__ static void load_vec(const float* p, float* f) {
    const uint4 v = ld_stream(p);
    f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
  }
  __device__ static void store_vec(float* p, const float* f) {
    *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
  }
};

// Adds elements [i, i + n) of `src` to acc[0 .. n).
template <typename T>
__device__ __forceinline__ void add_from(const typename Elem<T>::S* src, int64_t i, int n, float* acc) {
  constexpr int V = Elem<T>::kVec;
  const typename Elem<T>::S* p = src + i;
  if (n == V && (reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
    float f[V];
    Elem<T>::load_vec(p, f);
#pragma unroll
    for (int q = 0; q < V; ++q) acc[q] += f[q];
  } else {
    for (int q = 0; q < n; ++q) acc[q] += Elem<T>::load(p + q);
  }
}

template <typename T>
__device__ __forceinline__ void store_to(typename Elem<T>::S* dst, int64_t i, int n, const float* acc) {
  constexpr int V = Elem<T>::kVec;
  typename Elem<T>::S* p = dst + i;
  if (n == V && (reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
    Elem<T>::store_vec(p, acc);
  } else {
    for (int q = 0; q < n; ++q) Elem<T>::store(p + q, acc[q]);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void replica_items_kernel(typename Elem<T>::S* __restrict__ grads, int64_t P, int32_t C,
                                                            const int32_t* __restrict__ slot_offsets,
                                                            const int32_t* __restrict__ slots, int with_local,
                                                            int write_slots,
                                                            const int32_t* __restrict__ part_offsets,
                                                            const int64_t* __restrict__ part_ptrs,
                                                            const int32_t* __restrict__ out_offsets,
                                                            const int64_t* __restrict__ out_ptrs,
                                                            int32_t* __restrict__ status) {
  constexpr int V = Elem<T>::kVec;
  const int64_t item = blockIdx.y;
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V;
  if (i >= P) return;
  const int n = P - i < V ? (int)(P - i) : V;
  const int32_t s0 = slot_offsets[item], s1 = slot_offsets[item + 1];
  float acc[V];
#pragma unroll
  for (int q = 0; q < V; ++q) acc[q] = 0.f;
  if (with_local) {
    for (int32_t j = s0; j < s1; ++j) {
      const int32_t c = slots[j];
      if (c < 0 || c >= C) {
        atomicOr(status, 1);
        continue;
      }
      add_from<T>(grads + (int64_t)c * P, i, n, acc);
    }
  }
  if (part_offsets != nullptr) {
    for (int32_t j = part_offsets[item]; j < part_offsets[item + 1]; ++j)
      add_from<T>(reinterpret_cast<const typename Elem<T>::S*>(part_ptrs[j]), i, n, acc);
  }
  if (write_slots) {
    for (int32_t j = s0; j < s1; ++j) {
      const int32_t c = slots[j];
      if (c >= 0 && c < C) store_to<T>(grads + (int64_t)c * P, i, n, acc);
    }
  }
  if (out_offsets != nullptr) {
    for (int32_t j = out_offsets[item]; j < out_offsets[item + 1]; ++j)
      store_to<T>(reinterpret_cast<typename Elem<T>::S*>(out_ptrs[j]), i, n, acc);
  }
}

int launch_items(void* grads, int32_t dtype, int64_t P, int32_t C, int32_t n_items, const int32_t* slot_offsets,
                 const int32_t* slots, int with_local, int write_slots, const int32_t* part_offsets,
                 const int64_t* part_ptrs, const int32_t* out_offsets, const int64_t* out_ptrs, int32_t* status,
                 hipStream_t stream) {
  if (P < 0 || C < 0 || n_items < 0 || n_items > 65535) return PMX_ERR_ARG;
  if (dtype != PMX_DTYPE_BF16 && dtype != PMX_DTYPE_F16 && dtype != PMX_DTYPE_F32) return PMX_ERR_ARG;
  if (P == 0 || n_items == 0) return PMX_OK;
  if (!slot_offsets || !status || ((with_local || write_slots) && (!grads || (C > 0 && !slots)))) return PMX_ERR_ARG;
  if ((part_offsets == nullptr) != (part_ptrs == nullptr) || (out_offsets == nullptr) != (out_ptrs == nullptr))
    return PMX_ERR_ARG;
  const int V = dtype == PMX_DTYPE_F32 ? 4 : 8;
  const int64_t gx = (P + 256 * V - 1) / (256 * V);
  if (gx > 0x7fffffff) return PMX_ERR_SHAPE;
  const dim3 grid((unsigned)gx, (unsigned)n_items);
  if (dtype == PMX_DTYPE_BF16) {
    replica_items_kernel<EltBF16><<<grid, 256, 0, stream>>>(static_cast<bf16_t*>(grads), P, C, slot_offsets, slots,
                                                            with_local, write_slots, part_offsets, part_ptrs,
                                                            out_offsets, out_ptrs, status);
  } else if (dtype == PMX_DTYPE_F16) {
    replica_items_kernel<EltF16><<<grid, 256, 0, stream>>>(static_cast<bf16_t*>(grads), P, C, slot_offsets, slots,
                                                           with_local, write_slots, part_offsets, part_ptrs,
                                                           out_offsets, out_ptrs, status);
  } else {
    replica_items_kernel<float><<<grid, 256, 0, stream>>>(static_cast<float*>(grads), P, C, slot_offsets, slots,
                                                          with_local, write_slots, part_offsets, part_ptrs,
                                                          out_offsets, out_ptrs, status);
  }
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}

}  // namespace

extern "C" {

int pmx_replica_exchange_pack(const void* grads, int32_t dtype, int64_t P, int32_t C, int32_t n_items,
                              const int32_t* slot_offsets, const int32_t* slots, const int32_t* out_offsets,
                              const int64_t* out_ptrs, int32_t* status, pmx_stream_t stream) {
  if (out_offsets == nullptr || out_ptrs == nullptr) return PMX_ERR_ARG;
  return launch_items(const_cast<void*>(grads), dtype, P, C, n_items, slot_offsets, slots, 1, 0, nullptr, nullptr,
                      out_offsets, out_ptrs, status, stream);
}

int pmx_replica_exchange_unpack(void* grads, int32_t dtype, int64_t P, int32_t C, int32_t n_items,
                                const int32_t* slot_offsets, const int32_t* slots, int32_t with_local,
                                const int32_t* part_offsets, const int64_t* part_ptrs, const int32_t* out_offsets,
                                const int64_t* out_ptrs, int32_t* status, pmx_stream_t stream) {
  return launch_items(grads, dtype, P, C, n_items, slot_offsets, slots, with_local != 0, 1, part_offsets, part_ptrs,
                      out_offsets, out_ptrs, status, stream);
}

}  // extern "C"
