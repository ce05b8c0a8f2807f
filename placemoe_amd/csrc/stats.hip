// Route statistics for the PlaceMoE planner on gfx950: source-conditioned
// expert demand and pairwise co-selection counts of a routing sample,
// accumulated on the device so that a profiling window needs no host copy of
// the routes.
//
// One thread per token.  Counts are exact integers.  The demand table (S*E
// entries) is counted per block in LDS when it fits and added to the global
// table once per block and entry - with few experts every token would
// otherwise hit the same few counters.  The co-selection table (S*E*E) is
// counted the same way when it fits in 64 KB of LDS (one source row and up
// to 128 experts, say): every token's pairs then land in one small table and
// direct 64-bit atomics collide.  Larger co-selection tables take direct
// device-scope atomics; their entries are many and the updates of different
// tokens rarely collide.

#include "common.h"

namespace {

constexpr int kStatsMaxTopK = 32;
constexpr int kLdsDemand = 8192;     // demand entries counted in LDS per block
constexpr int kLdsAffinity = 16384;  // co-selection entries counted in LDS per block (dynamic LDS)
constexpr int kAffinityBlocks = 32;  // blocks (each over many tokens) when the co-selection table is in LDS

template <bool LDS_AFF>
__global__ __launch_bounds__(256) void route_stats_kernel(const int64_t* __restrict__ sel,
                                                          const int64_t* __restrict__ src, int32_t src_const,
                                                          int32_t S, int32_t E, int64_t T, int32_t K,
                                                          unsigned long long* __restrict__ demand,
                                                          unsigned long long* __restrict__ affinity,
                                                          int32_t* __restrict__ status) {
  __shared__ uint32_t lcount[kLdsDemand];
  extern __shared__ uint32_t laff[];  // S*E*E entries when LDS_AFF
  const int64_t SE = (int64_t)S * E;
  const int64_t SEE = SE * E;
  const bool lds = SE <= kLdsDemand;
  if (lds)
    for (int64_t i = threadIdx.x; i < SE; i += blockDim.x) lcount[i] = 0u;
  if constexpr (LDS_AFF)
    for (int64_t i = threadIdx.x; i < SEE; i += blockDim.x) laff[i] = 0u;
  __syncthreads();
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < T; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t s = src != nullptr ? src[t] : (int64_t)src_const;
    const int64_t* row = sel + t * K;
    bool ok = s >= 0 && s < S;
    for (int k = 0; k < K; ++k) ok = ok && row[k] >= 0 && row[k] < E;
    if (!ok) {
      // The whole token is skipped; the host reports the sample as invalid.
      atomicOr(status, 1);
      continue;
    }
    const int64_t base = s * E;
    for (int k = 0; k < K; ++k) {
      if (lds) atomicAdd(&lcount[base + row[k]], 1u);
      else atomicAdd(&demand[base + row[k]], 1ull);
    }
    // Unordered pairs k < k' of distinct experts, counted in both orders; a
    // pair of equal experts would land on the diagonal, which stays zero.
    for (int a = 0; a < K; ++a) {
      const int64_t ea = row[a];
      for (int b = a + 1; b < K; ++b) {
        const int64_t eb = row[b];
        if (ea == eb) continue;
        if constexpr (LDS_AFF) {
          atomicAdd(&laff[(base + ea) * E + eb], 1u);
          atomicAdd(&laff[(base + eb) * E + ea], 1u);
        } else {
          atomicAdd(&affinity[(base + ea) * E + eb], 1ull);
          atomicAdd(&affinity[(base + eb) * E + ea], 1ull);
        }
      }
    }
  }
  if (lds || LDS_AFF) __syncthreads();
  if (lds)
    for (int64_t i = threadIdx.x; i < SE; i += blockDim.x)
      if (lcount[i]) atomicAdd(&demand[i], (unsigned long long)lcount[i]);
  if constexpr (LDS_AFF)
    for (int64_t i = threadIdx.x; i < SEE; i += blockDim.x)
      if (laff[i]) atomicAdd(&affinity[i], (unsigned long long)laff[i]);
}

}  // namespace

extern "C" int pmx_route_statistics(const int64_t* sel, const int64_t* src, int32_t src_const, int32_t S,
                                    int32_t E, int64_t T, int32_t K, int64_t* demand, int64_t* affinity,
                                    int32_t* status, pmx_stream_t stream) {
  if (S <= 0 || E <= 0 || T < 0 || K <= 0 || K > kStatsMaxTopK) return PMX_ERR_ARG;
  if (!demand || !affinity || !status) return PMX_ERR_ARG;
  if ((int64_t)S * E * E > ((int64_t)1 << 40)) return PMX_ERR_SHAPE;
  if (T == 0) return PMX_OK;
  if (!sel) return PMX_ERR_ARG;
  const int64_t per_token = (T + 255) / 256;
  const int64_t SEE = (int64_t)S * E * E;
  auto* dem = reinterpret_cast<unsigned long long*>(demand);
  auto* aff = reinterpret_cast<unsigned long long*>(affinity);
  if (SEE <= kLdsAffinity && K > 1) {
    const unsigned blocks = (unsigned)(per_token < kAffinityBlocks ? per_token : kAffinityBlocks);
    route_stats_kernel<true><<<blocks, 256, (size_t)SEE * sizeof(uint32_t), stream>>>(sel, src, src_const, S, E, T,
                                                                                      K, dem, aff, status);
  } else {
    const unsigned blocks = (unsigned)(per_token < 4096 ? per_token : 4096);
    route_stats_kernel<false><<<blocks, 256, 0, stream>>>(sel, src, src_const, S, E, T, K, dem, aff, status);
  }
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}
