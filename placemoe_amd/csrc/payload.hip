// Rank-deduplicated expert-parallel payloads on gfx950: the per-rank halves
// of PlaceMoE's dispatch and combine around the all-to-all.
//
// Dispatch (sender): every assignment (t, k) goes to rank r = slot / slots_per_rank.
// A token sends its hidden row once per distinct target rank; the assignments
// travel as (unique ordinal within the rank, local slot, token) plus weight,
// ordered by (rank, token, k).  Both orders are stable counting sorts (the
// routing kernels of routing.hip): assignments by rank, and the first
// assignment of each (rank, token) pair by rank, with later duplicates parked
// in an extra bucket R that sorts last.
//
// Combine (receiver): weighted expert outputs of the received assignments,
// summed in fp32 per run of equal (source rank, source token) - the runs are
// contiguous because each sender's assignments arrive ordered by token.

#include "common.h"


namespace {

constexpr int kPayloadMaxTopK = 32;

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

// Per assignment: target rank, and that rank again if no earlier k of the
// same token targets it (else the parking bucket R).  Slots outside
// [0, R*L) are clamped and flagged.
__global__ __launch_bounds__(256) void payload_keys_kernel(const int32_t* __restrict__ phys, int64_t A, int32_t K,
                                                           int32_t R, int32_t L, int64_t* __restrict__ rank,
                                                           int64_t* __restrict__ first_rank,
                                                           int32_t* __restrict__ target_rank,
                                                           int32_t* __restrict__ status) {
  const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (a >= A) return;
  const int64_t row = a - a % K;
  const int32_t hi = R * L - 1;
  auto rank_of = [&](int64_t i) {
    int32_t p = phys[i];
    p = p < 0 ? 0 : (p > hi ? hi : p);
    return p / L;
  };
  const int32_t p = phys[a];
  if (p < 0 || p > hi) atomicOr(status, 1);
  const int32_t r = rank_of(a);
  bool first = true;
  for (int64_t i = row; i < a; ++i) first = first && rank_of(i) != r;
  rank[a] = r;
  first_rank[a] = first ? r : R;
  target_rank[a] = r;
}

// Per assignment: its metadata row and weight at its place in (rank, token,
// k) order, and, for the first assignment of a (rank, token) pair, the
// token of that unique row.
__global__ __launch_bounds__(256) void payload_meta_kernel(
    const int32_t* __restrict__ phys, const void* __restrict__ weights, int64_t A, int32_t K, int32_t R, int32_t L,
    const int64_t* __restrict__ rank, const int32_t* __restrict__ apos, const int32_t* __restrict__ upos,
    const int32_t* __restrict__ uoffsets, int32_t* __restrict__ send_meta, bf16_t* __restrict__ send_weights,
    int32_t* __restrict__ unique_tokens) {
  const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (a >= A) return;
  const int64_t t = a / K;
  const int64_t row = t * K;
  const int64_t r = rank[a];
  int64_t f = a;  // the first assignment of this token to rank r
  for (int64_t i = row; i < a; ++i) {
    if (rank[i] == r) {
      f = i;
      break;
    }
  }
  const int32_t u = upos[f];
  const int32_t hi = R * L - 1;
  int32_t p = phys[a];
  p = p < 0 ? 0 : (p > hi ? hi : p);
  const int64_t o = apos[a];
  send_meta[o * 3 + 0] = u - uoffsets[r];
  send_meta[o * 3 + 1] = p - (int32_t)r * L;
  send_meta[o * 3 + 2] = (int32_t)t;
  send_weights[o] = reinterpret_cast<const bf16_t*>(weights)[a];
  if (f == a) unique_tokens[u] = (int32_t)t;
}

// send_hidden[upos[a]] = hidden[t] for the first assignment a of each
// (rank, token) pair; one block per token.
__global__ __launch_bounds__(256) void payload_rows_kernel(const bf16_t* __restrict__ hidden,
                                                           const int64_t* __restrict__ first_rank,
                                                           const int32_t* __restrict__ upos, int32_t K, int32_t R,
                                                           int64_t H, bf16_t* __restrict__ send_hidden) {
  const int64_t t = blockIdx.x;
  const int64_t n8 = H / 8;
  const uint4* src = reinterpret_cast<const uint4*>(hidden + t * H);
  // The row is read once per chunk and stored to every rank that takes it.
  for (int64_t i = threadIdx.x; i < n8; i += blockDim.x) {
    const uint4 v = ld_stream(src + i);
    for (int k = 0; k < K; ++k) {
      const int64_t a = t * K + k;
      if (first_rank[a] == R) continue;
      reinterpret_cast<uint4*>(send_hidden + (int64_t)upos[a] * H)[i] = v;
    }
  }
}

__global__ void fill_kernel(int32_t* __restrict__ p, int32_t n) {
  const int32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

__global__ void copy_i32_kernel(const int32_t* __restrict__ src, int32_t* __restrict__ dst, int32_t n) {
  const int32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

// ---------------------------------------------------------------------------
// Combine aggregation
// ---------------------------------------------------------------------------

constexpr int kScanBlock = 1024;

// flag[a] = 1 where a run of equal (src_rank, src_token) starts; per-block
// sums of the flags.
__global__ __launch_bounds__(kScanBlock) void run_flags_kernel(const int32_t* __restrict__ src_rank,
                                                               const int32_t* __restrict__ src_token, int64_t N,
                                                               int32_t* __restrict__ flag,
                                                               int32_t* __restrict__ block_sum) {
  __shared__ int32_t red[kScanBlock / 64];
  const int64_t a = (int64_t)blockIdx.x * kScanBlock + threadIdx.x;
  int32_t f = 0;
  if (a < N) {
    f = (a == 0 || src_rank[a] != src_rank[a - 1] || src_token[a] != src_token[a - 1]) ? 1 : 0;
    flag[a] = f;
  }
  const uint64_t m = __ballot(f != 0);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = __popcll(m);
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t s = 0;
    for (int w = 0; w < kScanBlock / 64; ++w) s += red[w];
    block_sum[blockIdx.x] = s;
  }
}

// Exclusive scan of the block sums in one block; total -> *num_runs.
__global__ __launch_bounds__(kScanBlock) void scan_blocks_kernel(int32_t* __restrict__ block_sum, int64_t nblocks,
                                                                 int32_t* __restrict__ num_runs) {
  __shared__ int32_t sums[kScanBlock];
  __shared__ int32_t carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int64_t base = 0; base < nblocks; base += kScanBlock) {
    const int64_t i = base + threadIdx.x;
    const int32_t v = i < nblocks ? block_sum[i] : 0;
    sums[threadIdx.x] = v;
    __syncthreads();
    for (int off = 1; off < kScanBlock; off <<= 1) {
      const int32_t add = threadIdx.x >= off ? sums[threadIdx.x - off] : 0;
      __syncthreads();
      sums[threadIdx.x] += add;
      __syncthreads();
    }
    const int32_t c = carry;
    if (i < nblocks) block_sum[i] = c + sums[threadIdx.x] - v;
    __syncthreads();
    if (threadIdx.x == kScanBlock - 1) carry = c + sums[kScanBlock - 1];
    __syncthreads();
  }
  if (threadIdx.x == 0) *num_runs = carry;
}

// Run starts -> run_offsets[run] = a (and run_offsets[U] = N); runs per
// source rank, counted in LDS per block (up to kLdsRanks ranks) and added to
// the global counts once per block and rank: the ranks are sorted, so one
// block touches few of them, and a global atomic per run would serialise on
// R counters.
constexpr int kLdsRanks = 4096;

__global__ __launch_bounds__(kScanBlock) void run_offsets_kernel(const int32_t* __restrict__ flag,
                                                                 const int32_t* __restrict__ block_base,
                                                                 const int32_t* __restrict__ src_rank, int64_t N,
                                                                 int32_t R, const int32_t* __restrict__ num_runs,
                                                                 int32_t* __restrict__ run_offsets,
                                                                 int32_t* __restrict__ rank_runs,
                                                                 int32_t* __restrict__ status) {
  __shared__ int32_t wsum[kScanBlock / 64];
  __shared__ int32_t cnt[kLdsRanks];
  const bool lds = R <= kLdsRanks;
  if (lds)
    for (int i = threadIdx.x; i < R; i += kScanBlock) cnt[i] = 0;
  const int64_t a = (int64_t)blockIdx.x * kScanBlock + threadIdx.x;
  const int32_t f = a < N ? flag[a] : 0;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t m = __ballot(f != 0);
  if (lane == 0) wsum[w] = __popcll(m);
  __syncthreads();
  int32_t before = block_base[blockIdx.x];
  for (int i = 0; i < w; ++i) before += wsum[i];
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  if (f) {
    const int32_t run = before + __popcll(m & lt);
    run_offsets[run] = (int32_t)a;
    const int32_t r = src_rank[a];
    if (r >= 0 && r < R) {
      if (lds) atomicAdd(&cnt[r], 1);
      else atomicAdd(&rank_runs[r], 1);
    } else {
      atomicOr(status, 1);
    }
  }
  if (a == 0) run_offsets[*num_runs] = (int32_t)N;
  if (lds) {
    __syncthreads();
    for (int i = threadIdx.x; i < R; i += kScanBlock)
      if (cnt[i]) atomicAdd(&rank_runs[i], cnt[i]);
  }
}

// out[run] = bf16( sum_{a in run} fp32( bf16(Y[pos[a]] * w[a]) ) ); one block
// per potential run start (blocks past the number of runs exit).
template <class E>
__global__ __launch_bounds__(256) void run_combine_kernel(const bf16_t* __restrict__ Y,
                                                          const int32_t* __restrict__ pos,
                                                          const bf16_t* __restrict__ w,
                                                          const int32_t* __restrict__ run_offsets,
                                                          const int32_t* __restrict__ num_runs, int64_t H,
                                                          bf16_t* __restrict__ out) {
  const int64_t run = blockIdx.x;
  if (run >= *num_runs) return;
  const int32_t b = run_offsets[run], e = run_offsets[run + 1];
  const int64_t n8 = H / 8;
  for (int64_t i = threadIdx.x; i < n8; i += blockDim.x) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int32_t a = b; a < e; ++a) {
      float f[8];
      unpack8e<E>(ld_stream(reinterpret_cast<const uint4*>(Y + (int64_t)pos[a] * H) + i), f);
      const float wk = E::to_f32(w[a]);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += E::round(f[j] * wk);
    }
    reinterpret_cast<uint4*>(out + run * H)[i] = pack8e<E>(acc);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" {

size_t pmx_ep_payload_workspace_bytes(int64_t num_assign, int32_t num_ranks) {
  if (num_assign < 0 || num_ranks <= 0) return 0;
  const int64_t A = num_assign;
  size_t b = align256(pmx_route_ws_bytes(A, num_ranks + 1));
  b += 2 * align256((size_t)A * sizeof(int64_t));       // rank, first_rank
  b += 4 * align256((size_t)A * sizeof(int32_t));       // route phys outputs, apos, upos
  b += 2 * align256((size_t)(num_ranks + 2) * sizeof(int32_t));  // bucket counts, offsets
  b += 256;                                              // status
  return b;
}

int pmx_ep_dispatch_payload(const int32_t* phys, const void* hidden, const void* weights, int64_t T, int32_t K,
                            int64_t H, int32_t R, int32_t slots_per_rank, int32_t* assign_counts,
                            int32_t* assign_offsets, int32_t* unique_counts, int32_t* unique_offsets,
                            void* send_hidden, int32_t* unique_tokens, int32_t* send_meta, void* send_weights,
                            int32_t* target_rank, int32_t* status, void* workspace, size_t workspace_bytes,
                            pmx_stream_t stream) {
  if (T < 0 || K <= 0 || K > kPayloadMaxTopK || H < 0 || R <= 0 || slots_per_rank <= 0) return PMX_ERR_ARG;
  if ((int64_t)R * slots_per_rank > (int64_t)INT32_MAX) return PMX_ERR_SHAPE;
  if (H % 8) return PMX_ERR_SHAPE;
  if (!assign_counts || !assign_offsets || !unique_counts || !unique_offsets || !status || !workspace)
    return PMX_ERR_ARG;
  const int64_t A = T * K;
  if (A > (int64_t)INT32_MAX) return PMX_ERR_SHAPE;
  if (A > 0 && (!phys || !weights || !unique_tokens || !send_meta || !send_weights || !target_rank))
    return PMX_ERR_ARG;
  if (A > 0 && H > 0 && (!hidden || !send_hidden || !aligned16(hidden) || !aligned16(send_hidden)))
    return PMX_ERR_ARG;
  if (workspace_bytes < pmx_ep_payload_workspace_bytes(A, R)) return PMX_ERR_ARG;

  char* ws = reinterpret_cast<char*>(workspace);
  size_t off = 0;
  auto carve = [&](size_t bytes) {
    char* p = ws + off;
    off += align256(bytes);
    return p;
  };
  const size_t route_b = pmx_route_ws_bytes(A, R + 1);
  void* route_ws = carve(route_b);
  int64_t* rank = reinterpret_cast<int64_t*>(carve((size_t)A * sizeof(int64_t)));
  int64_t* first_rank = reinterpret_cast<int64_t*>(carve((size_t)A * sizeof(int64_t)));
  int32_t* rphys = reinterpret_cast<int32_t*>(carve((size_t)A * sizeof(int32_t)));
  int32_t* uphys = reinterpret_cast<int32_t*>(carve((size_t)A * sizeof(int32_t)));
  int32_t* apos = reinterpret_cast<int32_t*>(carve((size_t)A * sizeof(int32_t)));
  int32_t* upos = reinterpret_cast<int32_t*>(carve((size_t)A * sizeof(int32_t)));
  int32_t* ucounts = reinterpret_cast<int32_t*>(carve((size_t)(R + 2) * sizeof(int32_t)));
  int32_t* uoffsets = reinterpret_cast<int32_t*>(carve((size_t)(R + 2) * sizeof(int32_t)));

  if (A > 0) {
    payload_keys_kernel<<<(unsigned)((A + 255) / 256), 256, 0, stream>>>(phys, A, K, R, slots_per_rank, rank,
                                                                        first_rank, target_rank, status);
    PMX_LAUNCH_CHECK();
  }
  int rc = pmx_route_launch(rank, nullptr, nullptr, 0, 1, R, A, 1, R, rphys, assign_counts, assign_offsets, apos,
                            route_ws, route_b, stream);
  if (rc != PMX_OK) return rc;
  rc = pmx_route_launch(first_rank, nullptr, nullptr, 0, 1, R + 1, A, 1, R + 1, uphys, ucounts, uoffsets, upos,
                        route_ws, route_b, stream);
  if (rc != PMX_OK) return rc;
  copy_i32_kernel<<<(unsigned)((R + 256) / 256), 256, 0, stream>>>(ucounts, unique_counts, R);
  PMX_LAUNCH_CHECK();
  copy_i32_kernel<<<(unsigned)((R + 256) / 256), 256, 0, stream>>>(uoffsets, unique_offsets, R + 1);
  PMX_LAUNCH_CHECK();
  if (A == 0) return PMX_OK;
  payload_meta_kernel<<<(unsigned)((A + 255) / 256), 256, 0, stream>>>(
      phys, weights, A, K, R, slots_per_rank, rank, apos, upos, uoffsets, send_meta,
      static_cast<bf16_t*>(send_weights), unique_tokens);
  PMX_LAUNCH_CHECK();
  if (H > 0) {
    payload_rows_kernel<<<(unsigned)T, 256, 0, stream>>>(static_cast<const bf16_t*>(hidden), first_rank, upos, K, R,
                                                         H, static_cast<bf16_t*>(send_hidden));
    PMX_LAUNCH_CHECK();
  }
  return PMX_OK;
}

size_t pmx_ep_combine_workspace_bytes(int64_t num_recv) {
  if (num_recv < 0) return 0;
  const int64_t nblocks = (num_recv + kScanBlock - 1) / kScanBlock + 1;
  return align256((size_t)num_recv * sizeof(int32_t)) + align256((size_t)nblocks * sizeof(int32_t)) + 256;
}

}  // extern "C"

namespace {

template <class E>
int ep_combine_aggregate_t(const void* Y, const int32_t* pos, const void* w, const int32_t* src_rank,
                             const int32_t* src_token, int64_t N, int64_t H, int32_t R, void* out,
                             int32_t* run_offsets, int32_t* rank_runs, int32_t* num_runs, int32_t* status,
                             void* workspace, size_t workspace_bytes, pmx_stream_t stream) {
  if (N < 0 || H < 0 || R <= 0) return PMX_ERR_ARG;
  if (H % 8) return PMX_ERR_SHAPE;
  if (N > (int64_t)INT32_MAX) return PMX_ERR_SHAPE;
  if (!run_offsets || !rank_runs || !num_runs || !status || !workspace) return PMX_ERR_ARG;
  if (N > 0 && (!pos || !w || !src_rank || !src_token)) return PMX_ERR_ARG;
  if (N > 0 && H > 0 && (!Y || !out || !aligned16(Y) || !aligned16(out))) return PMX_ERR_ARG;
  if (workspace_bytes < pmx_ep_combine_workspace_bytes(N)) return PMX_ERR_ARG;
  int32_t* flag = reinterpret_cast<int32_t*>(workspace);
  int32_t* block_sum = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(workspace) +
                                                  align256((size_t)N * sizeof(int32_t)));
  const int64_t nblocks = (N + kScanBlock - 1) / kScanBlock;
  // Device-side zeroing (no memset nodes, so the path can sit in a graph).
  fill_kernel<<<(unsigned)((R + 255) / 256), 256, 0, stream>>>(rank_runs, R);
  PMX_LAUNCH_CHECK();
  fill_kernel<<<1, 64, 0, stream>>>(num_runs, 1);
  PMX_LAUNCH_CHECK();
  if (N == 0) {
    fill_kernel<<<1, 64, 0, stream>>>(run_offsets, 1);
    PMX_LAUNCH_CHECK();
    return PMX_OK;
  }
  run_flags_kernel<<<(unsigned)nblocks, kScanBlock, 0, stream>>>(src_rank, src_token, N, flag, block_sum);
  PMX_LAUNCH_CHECK();
  scan_blocks_kernel<<<1, kScanBlock, 0, stream>>>(block_sum, nblocks, num_runs);
  PMX_LAUNCH_CHECK();
  run_offsets_kernel<<<(unsigned)nblocks, kScanBlock, 0, stream>>>(flag, block_sum, src_rank, N, R, num_runs,
                                                                   run_offsets, rank_runs, status);
  PMX_LAUNCH_CHECK();
  if (H > 0) {
    run_combine_kernel<E><<<(unsigned)N, 256, 0, stream>>>(static_cast<const bf16_t*>(Y), pos,
                                                        static_cast<const bf16_t*>(w), run_offsets, num_runs, H,
                                                        static_cast<bf16_t*>(out));
    PMX_LAUNCH_CHECK();
  }
  return PMX_OK;
}

}  // namespace

extern "C" {

int pmx_ep_combine_aggregate(const void* Y, const int32_t* pos, const void* w, const int32_t* src_rank,
                             const int32_t* src_token, int64_t N, int64_t H, int32_t R, void* out,
                             int32_t* run_offsets, int32_t* rank_runs, int32_t* num_runs, int32_t* status,
                             void* workspace, size_t workspace_bytes, pmx_stream_t stream) {
  return ep_combine_aggregate_t<EltBF16>(Y, pos, w, src_rank, src_token, N, H, R, out, run_offsets, rank_runs,
                                        num_runs, status, workspace, workspace_bytes, stream);
}

int pmx_ep_combine_aggregate_f16(const void* Y, const int32_t* pos, const void* w, const int32_t* src_rank,
                                 const int32_t* src_token, int64_t N, int64_t H, int32_t R, void* out,
                                 int32_t* run_offsets, int32_t* rank_runs, int32_t* num_runs, int32_t* status,
                                 void* workspace, size_t workspace_bytes, pmx_stream_t stream) {
  return ep_combine_aggregate_t<EltF16>(Y, pos, w, src_rank, src_token, N, H, R, out, run_offsets, rank_runs,
                                        num_runs, status, workspace, workspace_bytes, stream);
}


}  // extern "C"
