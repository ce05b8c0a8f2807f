// Integer routing path (map -> histogram -> scan -> stable rank) and the
// bandwidth kernels that move rows (scatter, gather, weighted combine and
// its gradient, segment sum) for gfx950.
//
// Stable ranks are computed without atomics on the ordering: the flat
// assignment array is cut into chunks, one wave per chunk; a chunk's
// histogram row gives, after a column-wise exclusive scan, the first output
// position of every copy inside that chunk, and the wave then walks its chunk
// in 64-element segments, ranking equal values with wave ballots
// (match-any over the value bits) so that pos is identical to a stable
// argsort.

#include "common.h"

#include <string.h>

#include <mutex>

namespace {

constexpr int kRouteLdsMaxSlots = 8192;  // LDS counters up to this many copies
constexpr int kRouteMaxSlots = 1 << 24;
constexpr int kMaxTopK = 32;

struct RouteGeom {
  int64_t chunk;    // assignments per chunk (multiple of 64)
  int64_t nchunks;  // number of chunks (>= 1)
};

// Chunks of 512 assignments (eight 64-wide wave segments), so that a
// typical batch spreads over hundreds of one-wave blocks.  The chunk table
// (nchunks x C int32) is capped at 2^24 entries and 1024 rows; past that the
// chunks grow.
RouteGeom route_geom(int64_t A, int32_t C) {
  RouteGeom g;
  int64_t max_chunks = (int64_t(1) << 24) / C;
  if (max_chunks > 1024) max_chunks = 1024;
  if (max_chunks < 1) max_chunks = 1;
  g.chunk = 512;
  g.nchunks = (A + g.chunk - 1) / g.chunk;
  if (g.nchunks > max_chunks) {
    const int64_t per = (A + max_chunks - 1) / max_chunks;
    g.chunk = (per + 63) / 64 * 64;
    g.nchunks = (A + g.chunk - 1) / g.chunk;
  }
  if (g.nchunks < 1) g.nchunks = 1;
  return g;
}

constexpr size_t kStatusBytes = 256;

// Workspace: the status word (256 B), the chunk table, then one flag per
// chunk (its ids were clamped).
size_t route_ws_bytes(int64_t A, int32_t C) {
  RouteGeom g = route_geom(A, C);
  return kStatusBytes + (size_t)g.nchunks * (size_t)C * sizeof(int32_t) + (size_t)g.nchunks * sizeof(int32_t);
}

// Device-side fill (kept off hipMemsetAsync so the path can sit in a graph).
__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// One wave per chunk: phys = M[src, sel] (clamped, flagged) and the chunk
// histogram.  USE_LDS keeps the histogram in LDS, else in the chunk's own
// row of the global table (chunk-private, so plain atomics are exact).
template <bool USE_LDS>
__global__ __launch_bounds__(64) void route_hist_kernel(
    const int64_t* __restrict__ sel, const int64_t* __restrict__ M, const int64_t* __restrict__ src,
    int32_t src_const, int32_t S, int32_t E, int32_t K, int32_t C, int64_t A, int64_t chunk,
    int32_t* __restrict__ phys, int32_t* __restrict__ table, int32_t* __restrict__ flags) {
  extern __shared__ int32_t lds_hist[];
  const int lane = threadIdx.x;
  const int64_t ch = blockIdx.x;
  int32_t* row = table + ch * (int64_t)C;
  int32_t* hist = USE_LDS ? lds_hist : row;
  for (int c = lane; c < C; c += 64) hist[c] = 0;
  __syncthreads();
  const int64_t begin = ch * chunk;
  const int64_t end = begin + chunk < A ? begin + chunk : A;
  int bad = 0;
  for (int64_t a = begin + lane; a < end; a += 64) {
    int64_t e = sel[a];
    int64_t c;
    if (M != nullptr) {
      int64_t s = src != nullptr ? src[a / K] : (int64_t)src_const;
      if (s < 0 || s >= S) { bad = 1; s = s < 0 ? 0 : S - 1; }
      if (e < 0 || e >= E) { bad = 1; e = e < 0 ? 0 : E - 1; }
      c = M[s * E + e];
    } else {
      c = e;
    }
    if (c < 0 || c >= C) { bad = 1; c = c < 0 ? 0 : C - 1; }
    phys[a] = (int32_t)c;
    atomicAdd(&hist[c], 1);
  }
  __syncthreads();
  if (USE_LDS) {
    for (int c = lane; c < C; c += 64) row[c] = hist[c];
  }
  const bool any_bad = __ballot(bad) != 0;
  if (lane == 0) flags[ch] = any_bad ? 1 : 0;
}

// Single block: column-wise exclusive scan of the chunk table, turning
// histogram rows into per-chunk start positions, plus counts, offsets and the
// status word (the OR of the chunk flags).  With C < 1024 columns the 1024
// threads split each column into P = 1024 / C row ranges: the ranges are
// summed in parallel and their prefixes scanned in LDS, so a pass over the
// table costs nchunks / P dependent rows instead of nchunks.
__global__ __launch_bounds__(1024) void route_scan_kernel(int32_t* __restrict__ table, int64_t nchunks,
                                                          int32_t C, const int32_t* __restrict__ flags,
                                                          int32_t* __restrict__ counts,
                                                          int32_t* __restrict__ offsets,
                                                          int32_t* __restrict__ status) {
  __shared__ int32_t part[1024];  // per (range, column): range sum, then range start
  __shared__ int32_t sums[1024];
  __shared__ int32_t carry_sh;
  __shared__ int32_t bad_sh;
  const int tid = threadIdx.x;
  const int W = C < 1024 ? C : 1024;  // columns per pass
  int64_t P = 1024 / W;               // row ranges per column (1 when C >= 1024)
  if (P > nchunks) P = nchunks;
  const int64_t R = (nchunks + P - 1) / P;
  const int64_t p = tid / W;
  const int64_t r0 = p * R, r1 = r0 + R < nchunks ? r0 + R : nchunks;
  const bool ranged = C < 1024;  // one pass covers every column; `part` holds range starts
  if (tid == 0) bad_sh = 0;
  __syncthreads();
  {
    int32_t b = 0;
    for (int64_t r = tid; r < nchunks; r += 1024) b |= flags[r];
    if (b) atomicOr(&bad_sh, 1);
  }
  // Totals per column (and per range).
  for (int c0 = 0; c0 < C; c0 += W) {
    const int c = c0 + tid % W;
    int32_t run = 0;
    if (p < P && c < C) {
      int64_t r = r0;
      for (; r + 8 <= r1; r += 8) {
        int32_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = table[(r + j) * C + c];
#pragma unroll
        for (int j = 0; j < 8; ++j) run += v[j];
      }
      for (; r < r1; ++r) run += table[r * C + c];
    }
    if (ranged) part[tid] = run;
    else if (c < C) counts[c] = run;
  }
  __syncthreads();
  if (ranged && tid < C) {
    int32_t acc = 0;
    for (int64_t q = 0; q < P; ++q) {
      const int32_t v = part[q * W + tid];
      part[q * W + tid] = acc;
      acc += v;
    }
    counts[tid] = acc;
  }
  __syncthreads();
  if (tid == 0) carry_sh = 0;
  __syncthreads();
  for (int base = 0; base < C; base += 1024) {
    const int c = base + tid;
    const int32_t v = c < C ? counts[c] : 0;
    sums[tid] = v;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      int32_t add = tid >= off ? sums[tid - off] : 0;
      __syncthreads();
      sums[tid] += add;
      __syncthreads();
    }
    const int32_t carry = carry_sh;
    if (c < C) offsets[c] = carry + sums[tid] - v;
    __syncthreads();
    if (tid == 1023) carry_sh = carry + sums[1023];
    __syncthreads();
  }
  if (tid == 0) offsets[C] = carry_sh;
  __syncthreads();
  // Rows become start positions: offsets[c] + range start + running sum.
  for (int c0 = 0; c0 < C; c0 += W) {
    const int c = c0 + tid % W;
    if (p < P && c < C) {
      int32_t run = offsets[c] + (ranged ? part[tid] : 0);
      int64_t r = r0;
      for (; r + 8 <= r1; r += 8) {
        int32_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = table[(r + j) * C + c];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          table[(r + j) * C + c] = run;
          run += v[j];
        }
      }
      for (; r < r1; ++r) {
        const int32_t v = table[r * C + c];
        table[r * C + c] = run;
        run += v;
      }
    }
  }
  if (tid == 0) status[0] = bad_sh;
}

// One wave per chunk: stable rank of every assignment among equal copies.
template <bool USE_LDS>
__global__ __launch_bounds__(64) void route_rank_kernel(const int32_t* __restrict__ phys,
                                                         int32_t* __restrict__ table, int32_t C,
                                                         int64_t A, int64_t chunk, int nbits,
                                                         int32_t* __restrict__ pos) {
  extern __shared__ int32_t lds_cnt[];
  const int lane = threadIdx.x;
  const int64_t ch = blockIdx.x;
  int32_t* row = table + ch * (int64_t)C;
  int32_t* cnt = USE_LDS ? lds_cnt : row;
  if (USE_LDS) {
    for (int c = lane; c < C; c += 64) cnt[c] = row[c];
  }
  __syncthreads();
  const int64_t begin = ch * chunk;
  const int64_t end = begin + chunk < A ? begin + chunk : A;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t seg = begin; seg < end; seg += 64) {
    const int64_t a = seg + lane;
    const bool valid = a < end;
    const int32_t v = valid ? phys[a] : 0;
    uint64_t mask = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (v >> b) & 1;
      const uint64_t m = __ballot(bit);
      mask &= bit ? m : ~m;
    }
    int32_t base = 0;
    if (valid) {
      // The global-table counters are read and written by this wave only;
      // device-scope atomics keep every access at L2, in program order.
      base = USE_LDS ? cnt[v] : __hip_atomic_load(&cnt[v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (valid) {
      pos[a] = base + __popcll(mask & lt_mask);
      const int leader = 63 - __clzll(mask);
      if (lane == leader) {
        if (USE_LDS) cnt[v] = base + __popcll(mask);
        else __hip_atomic_store(&cnt[v], base + __popcll(mask), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
  }
}

// Row kernels launch one block per token and index rows with int32
// positions: T and T*K must fit in 31 bits.
inline bool rows_fit(int64_t T, int32_t K) { return T <= INT32_MAX / K; }

// `status` receives the routing status word; by default (NULL) it is the
// first word of the workspace.
int launch_route(const int64_t* sel, const int64_t* M, const int64_t* src, int32_t src_const,
                 int32_t S, int32_t E, int64_t A, int32_t K, int32_t C, int32_t* phys,
                 int32_t* counts, int32_t* offsets, int32_t* pos, void* workspace,
                 size_t workspace_bytes, hipStream_t stream, int32_t* status = nullptr) {
  if (C <= 0 || C > kRouteMaxSlots || A < 0 || K <= 0) return PMX_ERR_ARG;
  if (A > INT32_MAX) return PMX_ERR_SHAPE;  // positions and counts are int32
  if (!counts || !offsets || !workspace) return PMX_ERR_ARG;
  if (A > 0 && (!sel || !phys || !pos)) return PMX_ERR_ARG;
  if (M != nullptr && (S <= 0 || E <= 0)) return PMX_ERR_ARG;
  if (workspace_bytes < route_ws_bytes(A, C)) return PMX_ERR_ARG;
  if (status == nullptr) status = reinterpret_cast<int32_t*>(workspace);
  int32_t* table = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(workspace) + kStatusBytes);
  RouteGeom g = route_geom(A, C);
  int32_t* flags = table + g.nchunks * (int64_t)C;
  const bool lds = C <= kRouteLdsMaxSlots;
  const size_t lds_bytes = lds ? (size_t)C * sizeof(int32_t) : 0;
  if (A == 0) {
    // No assignments: the table is one zero row and its chunk flag (which
    // follows it) is clear; the scan still writes counts, offsets and the
    // status word.
    fill_i32_kernel<<<(unsigned)((C + 1 + 255) / 256), 256, 0, stream>>>(table, (int64_t)C + 1, 0);
  } else if (lds) {
    route_hist_kernel<true><<<(unsigned)g.nchunks, 64, lds_bytes, stream>>>(
        sel, M, src, src_const, S, E, K, C, A, g.chunk, phys, table, flags);
  } else {
    route_hist_kernel<false><<<(unsigned)g.nchunks, 64, 0, stream>>>(
        sel, M, src, src_const, S, E, K, C, A, g.chunk, phys, table, flags);
  }
  PMX_LAUNCH_CHECK();
  route_scan_kernel<<<1, 1024, 0, stream>>>(table, g.nchunks, C, flags, counts, offsets, status);
  PMX_LAUNCH_CHECK();
  if (A > 0) {
    int nbits = 1;
    while ((1 << nbits) < C) ++nbits;
    if (lds) {
      route_rank_kernel<true><<<(unsigned)g.nchunks, 64, lds_bytes, stream>>>(phys, table, C, A, g.chunk,
                                                                             nbits, pos);
    } else {
      route_rank_kernel<false><<<(unsigned)g.nchunks, 64, 0, stream>>>(phys, table, C, A, g.chunk, nbits,
                                                                      pos);
    }
    PMX_LAUNCH_CHECK();
  }
  return PMX_OK;
}

// ---------------------------------------------------------------------------
// Row movement.  One block per token row; 16-byte accesses when H % 8 == 0.
// ---------------------------------------------------------------------------

// Launch LAUNCH(KC) with KC = K for the common top-k values, else KC = 0 (the
// kernel's generic path, K read at run time).
#define PMX_DISPATCH_K(K, LAUNCH) \
  switch (K) {                    \
    case 1: LAUNCH(1); break;     \
    case 2: LAUNCH(2); break;     \
    case 4: LAUNCH(4); break;     \
    case 8: LAUNCH(8); break;     \
    default: LAUNCH(0); break;    \
  }

// One thread per 16-byte chunk of a row, whole waves, at most 512 threads:
// short blocks keep many rows in flight per CU (1024-thread blocks were
// slower on rows of 7168 bf16; there 384-512 threads gathered 7% faster than
// 256 and the other row kernels ran equal).
constexpr int kRowThreads = 512;
inline unsigned row_threads(int64_t H) {
  int64_t v = (H + 7) / 8;
  v = (v + 63) / 64 * 64;
  if (v < 64) v = 64;
  if (v > kRowThreads) v = kRowThreads;
  return (unsigned)v;
}

// STREAM_ST: streaming stores of the copies (top-1 only; see st_row).
template <bool VEC, bool STREAM_ST = false>
__global__ __launch_bounds__(kRowThreads) void scatter_rows_kernel(const bf16_t* __restrict__ X,
                                                           const int32_t* __restrict__ pos, int32_t K,
                                                           int64_t H, bf16_t* __restrict__ Xp,
                                                           int32_t* __restrict__ row_src,
                                                           const bf16_t* __restrict__ w,
                                                           bf16_t* __restrict__ row_w) {
  const int64_t t = blockIdx.x;
  const int32_t* p = pos + t * K;
  if (row_src != nullptr) {
    for (int32_t k = threadIdx.x; k < K; k += blockDim.x) {
      row_src[p[k]] = (int32_t)(t * K + k);
      if (row_w != nullptr) row_w[p[k]] = w[t * K + k];
    }
  }
  if (VEC) {
    const int64_t n8 = H / 8;
    const uint4* src = reinterpret_cast<const uint4*>(X + t * H);
    for (int64_t i = threadIdx.x; i < n8; i += blockDim.x) {
      const uint4 v = ld_stream(src + i);
      for (int k = 0; k < K; ++k) st_row<STREAM_ST>(reinterpret_cast<uint4*>(Xp + (int64_t)p[k] * H) + i, v);
    }
  } else {
    for (int64_t i = threadIdx.x; i < H; i += blockDim.x) {
      const bf16_t v = X[t * H + i];
      for (int k = 0; k < K; ++k) Xp[(int64_t)p[k] * H + i] = v;
    }
  }
}

// Top-1 row map: row_src[pos[t]] = t and, with w, row_w[pos[t]] = w[t] (one
// thread per token; a pos outside [0, T) is skipped).
__global__ __launch_bounds__(256) void invert_top1_kernel(const int32_t* __restrict__ pos, const bf16_t* __restrict__ w,
                                                          int64_t T, int32_t* __restrict__ row_src,
                                                          bf16_t* __restrict__ row_w) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const int32_t r = pos[t];
  if (r < 0 || r >= T) return;
  row_src[r] = (int32_t)t;
  if (row_w != nullptr) row_w[r] = w[t];
}

// The top-1 permute in the rows' storage order: block r copies token row
// row_src[r] of X to row r of Xp (written front to back, streaming stores;
// a token outside [0, T) gives a zero row).  Against the token-order walk,
// which reads X in order and writes the rows at random: 6.1 against 5.25
// TB/s on the DeepSeek-V3-shape rows (65536 x 7168), bit-identical.
__global__ __launch_bounds__(kRowThreads) void gather_rows_by_src_kernel(const bf16_t* __restrict__ X,
                                                                         const int32_t* __restrict__ row_src,
                                                                         int64_t T, int64_t H,
                                                                         bf16_t* __restrict__ Xp) {
  const int64_t r = blockIdx.x;
  const int64_t t = row_src[r];
  const bool ok = t >= 0 && t < T;
  const int64_t n8 = H / 8;
  const uint4* src = reinterpret_cast<const uint4*>(X + (ok ? t : 0) * H);
  uint4* dst = reinterpret_cast<uint4*>(Xp + r * H);
  for (int64_t i = threadIdx.x; i < n8; i += blockDim.x) st_stream(dst + i, ok ? ld_stream(src + i) : make_uint4(0, 0, 0, 0));
}

// out[t] = bf16( sum_k fp32(term_k) ), term_k = Y[pos] or bf16(Y[pos] * w).
// KC > 0: K == KC at compile time; the K row loads of a chunk are issued
// together, then summed in k order (the same order as the generic path).
template <class E, bool VEC, bool WEIGHTED, int KC = 0>
__global__ __launch_bounds__(kRowThreads) void gather_rows_kernel(const bf16_t* __restrict__ Y,
                                                           const int32_t* __restrict__ pos,
                                                           const bf16_t* __restrict__ w, int32_t K,
                                                           int64_t H, bf16_t* __restrict__ out) {
  const int64_t t = blockIdx.x;
  const int32_t* p = pos + t * K;
  if constexpr (VEC && KC > 0) {
    const int64_t n8 = H / 8;
    int64_t rows[KC];
    float wk[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      rows[k] = (int64_t)p[k] * H;
      wk[k] = WEIGHTED ? E::to_f32(w[t * KC + k]) : 1.f;
    }
    for (int64_t i = threadIdx.x; i < n8; i += blockDim.x) {
      uint4 v[KC];
#pragma unroll
      for (int k = 0; k < KC; ++k) v[k] = ld_stream(reinterpret_cast<const uint4*>(Y + rows[k]) + i);
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        float f[8];
        unpack8e<E>(v[k], f);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += WEIGHTED ? E::round(f[j] * wk[k]) : f[j];
      }
      reinterpret_cast<uint4*>(out + t * H)[i] = pack8e<E>(acc);
    }
  } else if (VEC) {
    const int64_t n8 = H / 8;
    for (int64_t i = threadIdx.x; i < n8; i += blockDim.x) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int k = 0; k < K; ++k) {
        const uint4 v = ld_stream(reinterpret_cast<const uint4*>(Y + (int64_t)p[k] * H) + i);
        float f[8];
        unpack8e<E>(v, f);
        if (WEIGHTED) {
          const float wk = E::to_f32(w[t * K + k]);
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[j] += E::round(f[j] * wk);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[j] += f[j];
        }
      }
      reinterpret_cast<uint4*>(out + t * H)[i] = pack8e<E>(acc);
    }
  } else {
    for (int64_t i = threadIdx.x; i < H; i += blockDim.x) {
      float acc = 0.f;
      for (int k = 0; k < K; ++k) {
        const float f = E::to_f32(Y[(int64_t)p[k] * H + i]);
        if (WEIGHTED) acc += E::round(f * E::to_f32(w[t * K + k]));
        else acc += f;
      }
      out[t * H + i] = (bf16_t)E::from_f32(acc);
    }
  }
}

// KC > 0: K == KC at compile time; a chunk's K loads of Y are issued together.
// Top-1 (KC == 1) stores dY with streaming stores (see st_row).  dout and Y
// are read with streaming loads: plain loads measured 1.5-3% faster on
// isolated buffers but 11% slower inside the layer step (Qwen3 shape).
template <class E, bool VEC, int KC = 0>
__global__ __launch_bounds__(kRowThreads) void combine_bwd_kernel(const bf16_t* __restrict__ dout,
                                                           const bf16_t* __restrict__ Y,
                                                           const int32_t* __restrict__ pos,
                                                           const bf16_t* __restrict__ w, int32_t K,
                                                           int64_t H, bf16_t* __restrict__ dY,
                                                           bf16_t* __restrict__ dw) {
  __shared__ float red[kRowThreads / 64][kMaxTopK];
  const int64_t t = blockIdx.x;
  const int32_t* p = pos + t * K;
  float part[kMaxTopK];
#pragma unroll
  for (int k = 0; k < kMaxTopK; ++k) part[k] = 0.f;
  if constexpr (VEC && KC > 0) {
    const int64_t n8 = H / 8;
    int64_t rows[KC];
    float wk[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      rows[k] = (int64_t)p[k] * H;
      wk[k] = E::to_f32(w[t * KC + k]);
    }
    for (int64_t i = threadIdx.x; i < n8; i += blockDim.x) {
      float d[8];
      unpack8e<E>(ld_stream(reinterpret_cast<const uint4*>(dout + t * H) + i), d);
      uint4 yv[KC];
#pragma unroll
      for (int k = 0; k < KC; ++k) yv[k] = ld_stream(reinterpret_cast<const uint4*>(Y + rows[k]) + i);
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        float g[8], y[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) g[j] = d[j] * wk[k];
        st_row<KC == 1>(reinterpret_cast<uint4*>(dY + rows[k]) + i, pack8e<E>(g));
        unpack8e<E>(yv[k], y);
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) s += E::round(d[j] * y[j]);
        part[k] += s;
      }
    }
  } else if (VEC) {
    const int64_t n8 = H / 8;
    for (int64_t i = threadIdx.x; i < n8; i += blockDim.x) {
      float d[8];
      unpack8e<E>(ld_stream(reinterpret_cast<const uint4*>(dout + t * H) + i), d);
#pragma unroll
      for (int k = 0; k < kMaxTopK; ++k) {
        if (k < K) {
          const int64_t row = p[k];
          const float wk = E::to_f32(w[t * K + k]);
          float g[8], y[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) g[j] = d[j] * wk;
          reinterpret_cast<uint4*>(dY + row * H)[i] = pack8e<E>(g);
          unpack8e<E>(ld_stream(reinterpret_cast<const uint4*>(Y + row * H) + i), y);
          float s = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) s += E::round(d[j] * y[j]);
          part[k] += s;
        }
      }
    }
  } else {
    for (int64_t i = threadIdx.x; i < H; i += blockDim.x) {
      const float d = E::to_f32(dout[t * H + i]);
#pragma unroll
      for (int k = 0; k < kMaxTopK; ++k) {
        if (k < K) {
          const int64_t row = p[k];
          const float wk = E::to_f32(w[t * K + k]);
          dY[row * H + i] = (bf16_t)E::from_f32(d * wk);
          part[k] += E::round(d * E::to_f32(Y[row * H + i]));
        }
      }
    }
  }
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int nwaves = blockDim.x / 64;
#pragma unroll
  for (int k = 0; k < kMaxTopK; ++k) {
    if (k < K) {
      const float s = wave_sum(part[k]);
      if (lane == 0) red[wave][k] = s;
    }
  }
  __syncthreads();
  if (threadIdx.x < (unsigned)K) {
    float s = 0.f;
    for (int wv = 0; wv < nwaves; ++wv) s += red[wv][threadIdx.x];
    dw[t * K + threadIdx.x] = (bf16_t)E::from_f32(s);
  }
}

// Top-1 combine gradient with one wave per token: dY[pos[t]] = bf16(dout[t] * w[t])
// and dw[t] = bf16(sum_h fp32(bf16(dout[t,h] * Y[pos[t],h]))), the sum kept in
// lane partials and reduced across the wave (no LDS, no block barrier).  Each
// lane moves UNR 16-byte chunks of both rows per pass, all loads first; with
// UNR = 14 a 7168-wide row takes one pass (measured 5.61 TB/s against 5.48
// with two passes of 7; 8 tokens per block or plain stores of dY were no
// faster).
template <class E, int UNR>
__global__ __launch_bounds__(256) void combine_bwd_top1_kernel(const bf16_t* __restrict__ dout,
                                                               const bf16_t* __restrict__ Y,
                                                               const int32_t* __restrict__ pos,
                                                               const bf16_t* __restrict__ w, int64_t T, int64_t H,
                                                               bf16_t* __restrict__ dY, bf16_t* __restrict__ dw) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (t >= T) return;
  const int64_t row = (int64_t)pos[t] * H;
  const float wk = E::to_f32(w[t]);
  const int64_t n8 = H / 8;
  const uint4* d_row = reinterpret_cast<const uint4*>(dout + t * H);
  const uint4* y_row = reinterpret_cast<const uint4*>(Y + row);
  uint4* g_row = reinterpret_cast<uint4*>(dY + row);
  float part = 0.f;
  for (int64_t base = lane; base < n8; base += 64 * UNR) {
    uint4 dv[UNR], yv[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t i = base + 64 * u;
      if (i < n8) {
        dv[u] = ld_stream(d_row + i);
        yv[u] = ld_stream(y_row + i);
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t i = base + 64 * u;
      if (i < n8) {
        float d[8], y[8], g[8];
        unpack8e<E>(dv[u], d);
        unpack8e<E>(yv[u], y);
#pragma unroll
        for (int j = 0; j < 8; ++j) g[j] = d[j] * wk;
        st_stream(g_row + i, pack8e<E>(g));
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) s += E::round(d[j] * y[j]);
        part += s;
      }
    }
  }
  part = wave_sum(part);
  if (lane == 0) dw[t] = (bf16_t)E::from_f32(part);
}

// Top-1 combine gradient in the rows' storage order: wave r handles row r of
// Y and dY (read and written front to back) and gathers its token's dout row.
// On the DeepSeek-V3-shape rows (65536 x 7168, a random row order) this moves
// 5.8 TB/s against 5.2 TB/s for the token-order walk (combine_bwd_top1_kernel),
// whose Y reads and dY writes jump between rows; results are bit-identical
// (the same arithmetic per element and the same per-row sum order).
template <class E, int UNR>
__global__ __launch_bounds__(256) void combine_bwd_top1_rows_kernel(const bf16_t* __restrict__ dout,
                                                                    const bf16_t* __restrict__ Y,
                                                                    const int32_t* __restrict__ row_token,
                                                                    const bf16_t* __restrict__ w, int64_t T,
                                                                    int64_t H, bf16_t* __restrict__ dY,
                                                                    bf16_t* __restrict__ dw) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (r >= T) return;
  const int64_t t = row_token[r];
  const bool ok = t >= 0 && t < T;
  const float wk = ok ? E::to_f32(w[t]) : 0.f;
  const int64_t n8 = H / 8;
  const uint4* d_row = reinterpret_cast<const uint4*>(dout + (ok ? t : 0) * H);
  const uint4* y_row = reinterpret_cast<const uint4*>(Y + r * H);
  uint4* g_row = reinterpret_cast<uint4*>(dY + r * H);
  float part = 0.f;
  for (int64_t base = lane; base < n8; base += 64 * UNR) {
    uint4 dv[UNR], yv[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t i = base + 64 * u;
      if (i < n8) {
        dv[u] = ok ? ld_stream(d_row + i) : make_uint4(0, 0, 0, 0);
        yv[u] = ld_stream(y_row + i);
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t i = base + 64 * u;
      if (i < n8) {
        float d[8], y[8], g[8];
        unpack8e<E>(dv[u], d);
        unpack8e<E>(yv[u], y);
#pragma unroll
        for (int j = 0; j < 8; ++j) g[j] = d[j] * wk;
        st_stream(g_row + i, pack8e<E>(g));
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) s += E::round(d[j] * y[j]);
        part += s;
      }
    }
  }
  part = wave_sum(part);
  if (lane == 0 && ok) dw[t] = (bf16_t)E::from_f32(part);
}

// order[pos[i]] = i : the inverse of the stable scatter index.
__global__ void invert_kernel(const int32_t* __restrict__ pos, int64_t N, int32_t* __restrict__ order) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < N) order[pos[i]] = (int32_t)i;
}

// out[r] = sum_{j in [off[r], off[r+1])} src[order[j]]  (fp32, bf16 store).
template <class E, bool VEC>
__global__ __launch_bounds__(kRowThreads) void segment_rows_kernel(const bf16_t* __restrict__ src,
                                                           const int32_t* __restrict__ order,
                                                           const int32_t* __restrict__ off, int64_t H,
                                                           bf16_t* __restrict__ out) {
  const int64_t r = blockIdx.x;
  const int32_t b = off[r], e = off[r + 1];
  if (VEC) {
    const int64_t n8 = H / 8;
    for (int64_t i = threadIdx.x; i < n8; i += blockDim.x) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int32_t j = b; j < e; ++j) {
        float f[8];
        unpack8e<E>(ld_stream(reinterpret_cast<const uint4*>(src + (int64_t)order[j] * H) + i), f);
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[q] += f[q];
      }
      reinterpret_cast<uint4*>(out + r * H)[i] = pack8e<E>(acc);
    }
  } else {
    for (int64_t i = threadIdx.x; i < H; i += blockDim.x) {
      float acc = 0.f;
      for (int32_t j = b; j < e; ++j) acc += E::to_f32(src[(int64_t)order[j] * H + i]);
      out[r * H + i] = (bf16_t)E::from_f32(acc);
    }
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

int pmx_route_launch(const int64_t* sel, const int64_t* M, const int64_t* src, int32_t src_const, int32_t S,
                     int32_t E, int64_t A, int32_t K, int32_t C, int32_t* phys, int32_t* counts, int32_t* offsets,
                     int32_t* pos, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return launch_route(sel, M, src, src_const, S, E, A, K, C, phys, counts, offsets, pos, workspace, workspace_bytes,
                      stream);
}

size_t pmx_route_ws_bytes(int64_t A, int32_t C) { return route_ws_bytes(A, C); }

// ---------------------------------------------------------------------------
// Device scratch of pmx_route_noalloc: the routing chunk table lives in a
// static device array instead of a caller workspace.  Each GPU holds its own
// copy until the process ends.  On the host the array's name is only a
// stand-in, never a device address: host code uses the per-device address
// that hipGetSymbolAddress returns, taken once per device.
// ---------------------------------------------------------------------------

constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up on the first call on
// that device (with that device current) and kept for later calls.
int scratch_for_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return PMX_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return PMX_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PMX_OK;
}

}  // namespace

extern "C" {

const char* pmx_version(void) { return "placemoe_amd 0.1.0 gfx950"; }

const char* pmx_error_string(int code) {
  switch (code) {
    case PMX_OK: return "ok";
    case PMX_ERR_HIP: return "HIP runtime error";
    case PMX_ERR_ARG: return "invalid argument";
    case PMX_ERR_SHAPE: return "unsupported shape";
    case PMX_ERR_RANGE: return "index out of range";
    default: return "unknown error";
  }
}

size_t pmx_route_workspace_bytes(int64_t num_assign, int32_t num_slots) {
  if (num_assign < 0 || num_slots <= 0) return 0;
  return route_ws_bytes(num_assign, num_slots);
}

int pmx_route(const int64_t* sel, const int64_t* M, const int64_t* src, int32_t src_const, int32_t S,
              int32_t E, int64_t T, int32_t K, int32_t C, int32_t* phys, int32_t* counts,
              int32_t* offsets, int32_t* pos, void* workspace, size_t workspace_bytes,
              pmx_stream_t stream) {
  if (T < 0 || K <= 0) return PMX_ERR_ARG;
  if (M == nullptr && src != nullptr) return PMX_ERR_ARG;
  if (T > INT32_MAX / K) return PMX_ERR_SHAPE;
  return launch_route(sel, M, src, src_const, S, E, T * K, K, C, phys, counts, offsets, pos, workspace,
                      workspace_bytes, stream);
}

int pmx_route_noalloc(const int64_t* sel, const int64_t* M, const int64_t* src, int32_t src_const, int32_t S,
                      int32_t E, int64_t T, int32_t K, int32_t C, int32_t* phys, int32_t* counts,
                      int32_t* offsets, int32_t* pos, int32_t* status, pmx_stream_t stream) {
  if (T < 0 || K <= 0 || C <= 0) return PMX_ERR_ARG;
  if (M == nullptr && src != nullptr) return PMX_ERR_ARG;
  if (T > INT32_MAX / K) return PMX_ERR_SHAPE;
  // The chunk table must fit the static scratch: refuse before any launch.
  if (route_ws_bytes(T * K, C) > kNoAllocScratchBytes) return PMX_ERR_SHAPE;
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc != PMX_OK) return rc;
  int32_t* st = status != nullptr ? status : static_cast<int32_t*>(ws);
  return launch_route(sel, M, src, src_const, S, E, T * K, K, C, phys, counts, offsets, pos, ws,
                      kNoAllocScratchBytes, stream, st);
}

int pmx_route_status(const void* workspace, int32_t* status_host, pmx_stream_t stream) {
  if (!workspace || !status_host) return PMX_ERR_ARG;
  hipError_t e = hipMemcpyAsync(status_host, workspace, sizeof(int32_t), hipMemcpyDeviceToHost, stream);
  if (e != hipSuccess) return PMX_ERR_HIP;
  return pmx_status(hipStreamSynchronize(stream));
}

int pmx_moe_scatter(const void* X, const int32_t* pos, int64_t T, int32_t K, int64_t H, void* Xp,
                    pmx_stream_t stream) {
  return pmx_moe_scatter_src(X, pos, nullptr, T, K, H, Xp, nullptr, nullptr, stream);
}

int pmx_moe_scatter_src(const void* X, const int32_t* pos, const void* w, int64_t T, int32_t K, int64_t H,
                        void* Xp, int32_t* row_src, void* row_w, pmx_stream_t stream) {
  if (T < 0 || K <= 0 || H < 0) return PMX_ERR_ARG;
  if (!rows_fit(T, K)) return PMX_ERR_SHAPE;
  if ((w != nullptr) != (row_w != nullptr) || (row_w != nullptr && row_src == nullptr)) return PMX_ERR_ARG;
  if (T == 0 || (H == 0 && row_src == nullptr)) return PMX_OK;
  if (!X || !pos || !Xp) return PMX_ERR_ARG;
  const unsigned th = row_threads(H);
  const bf16_t* wb = static_cast<const bf16_t*>(w);
  bf16_t* rw = static_cast<bf16_t*>(row_w);
  if (H % 8 == 0 && aligned16(X) && aligned16(Xp)) {
    if (K == 1 && row_src != nullptr) {
      // top-1 with the row map: the map first (every row -1, then the rows
      // pos names), then the rows in storage order
      fill_i32_kernel<<<(unsigned)((T + 255) / 256), 256, 0, stream>>>(row_src, T, -1);
      PMX_LAUNCH_CHECK();
      invert_top1_kernel<<<(unsigned)((T + 255) / 256), 256, 0, stream>>>(pos, wb, T, row_src, rw);
      PMX_LAUNCH_CHECK();
      gather_rows_by_src_kernel<<<(unsigned)T, th, 0, stream>>>((const bf16_t*)X, row_src, T, H, (bf16_t*)Xp);
    } else if (K == 1) {
      scatter_rows_kernel<true, true><<<(unsigned)T, th, 0, stream>>>((const bf16_t*)X, pos, K, H, (bf16_t*)Xp,
                                                                      row_src, wb, rw);
    } else {
      scatter_rows_kernel<true><<<(unsigned)T, th, 0, stream>>>((const bf16_t*)X, pos, K, H, (bf16_t*)Xp, row_src,
                                                                wb, rw);
    }
  } else {
    scatter_rows_kernel<false><<<(unsigned)T, th, 0, stream>>>((const bf16_t*)X, pos, K, H, (bf16_t*)Xp, row_src,
                                                               wb, rw);
  }
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}

}  // extern "C"

namespace {

template <class E>
int moe_gather_t(const void* Y, const int32_t* pos, int64_t T, int32_t K, int64_t H, void* out,
                   pmx_stream_t stream) {
  if (T < 0 || K <= 0 || H < 0) return PMX_ERR_ARG;
  if (!rows_fit(T, K)) return PMX_ERR_SHAPE;
  if (T == 0 || H == 0) return PMX_OK;
  if (!Y || !pos || !out) return PMX_ERR_ARG;
  const unsigned th = row_threads(H);
  if (H % 8 == 0 && aligned16(Y) && aligned16(out)) {
#define PMX_GATHER(KC)                                                                                  \
  gather_rows_kernel<E, true, false, KC><<<(unsigned)T, th, 0, stream>>>((const bf16_t*)Y, pos, nullptr, K, H, \
                                                                     (bf16_t*)out)
    PMX_DISPATCH_K(K, PMX_GATHER);
#undef PMX_GATHER
  } else {
    gather_rows_kernel<E, false, false><<<(unsigned)T, th, 0, stream>>>((const bf16_t*)Y, pos, nullptr, K, H,
                                                                    (bf16_t*)out);
  }
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}

template <class E>
int combine_fwd_t(const void* Y, const int32_t* pos, const void* w, int64_t T, int32_t K, int64_t H,
                    void* out, pmx_stream_t stream) {
  if (T < 0 || K <= 0 || H < 0) return PMX_ERR_ARG;
  if (!rows_fit(T, K)) return PMX_ERR_SHAPE;
  if (T == 0 || H == 0) return PMX_OK;
  if (!Y || !pos || !w || !out) return PMX_ERR_ARG;
  const unsigned th = row_threads(H);
  if (H % 8 == 0 && aligned16(Y) && aligned16(out)) {
#define PMX_COMBINE(KC)                                                                               \
  gather_rows_kernel<E, true, true, KC><<<(unsigned)T, th, 0, stream>>>((const bf16_t*)Y, pos, (const bf16_t*)w, \
                                                                    K, H, (bf16_t*)out)
    PMX_DISPATCH_K(K, PMX_COMBINE);
#undef PMX_COMBINE
  } else {
    gather_rows_kernel<E, false, true><<<(unsigned)T, th, 0, stream>>>((const bf16_t*)Y, pos, (const bf16_t*)w,
                                                                   K, H, (bf16_t*)out);
  }
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}

template <class E>
int combine_bwd_top1_rows_t(const void* dout, const void* Y, const int32_t* row_token, const void* w,
                              int64_t T, int64_t H, void* dY, void* dw, pmx_stream_t stream) {
  if (T < 0 || H < 0) return PMX_ERR_ARG;
  if (!rows_fit(T, 1)) return PMX_ERR_SHAPE;
  if (T == 0) return PMX_OK;
  if (!dout || !Y || !row_token || !w || !dY || !dw) return PMX_ERR_ARG;
  if (H % 8 || !aligned16(dout) || !aligned16(Y) || !aligned16(dY)) return PMX_ERR_SHAPE;
  const int64_t blocks = (T + 3) / 4;  // a wave per row, 4 rows per block
  if (blocks > 0x7fffffff) return PMX_ERR_SHAPE;
  combine_bwd_top1_rows_kernel<E, 14><<<(unsigned)blocks, 256, 0, stream>>>(
      (const bf16_t*)dout, (const bf16_t*)Y, row_token, (const bf16_t*)w, T, H, (bf16_t*)dY, (bf16_t*)dw);
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}

template <class E>
int combine_bwd_t(const void* dout, const void* Y, const int32_t* pos, const void* w, int64_t T,
                    int32_t K, int64_t H, void* dY, void* dw, pmx_stream_t stream) {
  if (T < 0 || K <= 0 || H < 0) return PMX_ERR_ARG;
  if (K > kMaxTopK) return PMX_ERR_ARG;
  if (!rows_fit(T, K)) return PMX_ERR_SHAPE;
  if (T == 0) return PMX_OK;
  if (!dout || !Y || !pos || !w || !dY || !dw) return PMX_ERR_ARG;
  const unsigned th = row_threads(H);
  if (K == 1 && H % 8 == 0 && H >= 2048 && aligned16(dout) && aligned16(Y) && aligned16(dY)) {
    // top-1 rows of at least 2048 columns: a wave per token (4 tokens per block)
    const int64_t blocks = (T + 3) / 4;
    if (blocks > 0x7fffffff) return PMX_ERR_SHAPE;
    combine_bwd_top1_kernel<E, 14><<<(unsigned)blocks, 256, 0, stream>>>(
        (const bf16_t*)dout, (const bf16_t*)Y, pos, (const bf16_t*)w, T, H, (bf16_t*)dY, (bf16_t*)dw);
    PMX_LAUNCH_CHECK();
    return PMX_OK;
  }
  if (H % 8 == 0 && aligned16(dout) && aligned16(Y) && aligned16(dY)) {
#define PMX_COMBINE_BWD(KC)                                                                            \
  combine_bwd_kernel<E, true, KC><<<(unsigned)T, th, 0, stream>>>((const bf16_t*)dout, (const bf16_t*)Y, pos, \
                                                              (const bf16_t*)w, K, H, (bf16_t*)dY, (bf16_t*)dw)
    PMX_DISPATCH_K(K, PMX_COMBINE_BWD);
#undef PMX_COMBINE_BWD
  } else {
    combine_bwd_kernel<E, false><<<(unsigned)T, th, 0, stream>>>((const bf16_t*)dout, (const bf16_t*)Y, pos,
                                                             (const bf16_t*)w, K, H, (bf16_t*)dY,
                                                             (bf16_t*)dw);
  }
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}

template <class E>
int segment_sum_t(const void* source, const int64_t* index, int64_t N, int64_t H, int64_t num_rows,
                    void* out, void* workspace, size_t workspace_bytes, pmx_stream_t stream) {
  if (N < 0 || H < 0 || num_rows < 0) return PMX_ERR_ARG;
  if (num_rows == 0) return N == 0 ? PMX_OK : PMX_ERR_ARG;
  if (num_rows > kRouteMaxSlots || N > INT32_MAX) return PMX_ERR_SHAPE;
  if (!out || !workspace) return PMX_ERR_ARG;
  if (N > 0 && (!source || !index)) return PMX_ERR_ARG;
  if (workspace_bytes < pmx_segment_sum_workspace_bytes(N, num_rows)) return PMX_ERR_ARG;
  const int32_t R = (int32_t)num_rows;
  char* ws = reinterpret_cast<char*>(workspace);
  size_t route_b = (route_ws_bytes(N, R) + 255) / 256 * 256;
  auto carve = [&](size_t n_int) {
    int32_t* p = reinterpret_cast<int32_t*>(ws + route_b);
    route_b += (n_int * sizeof(int32_t) + 255) / 256 * 256;
    return p;
  };
  int32_t* phys = carve((size_t)N);
  int32_t* pos = carve((size_t)N);
  int32_t* order = carve((size_t)N);
  int32_t* counts = carve((size_t)R);
  int32_t* offsets = carve((size_t)R + 1);
  int rc = launch_route(index, nullptr, nullptr, 0, 1, R, N, 1, R, phys, counts, offsets, pos, workspace,
                        route_ws_bytes(N, R), stream);
  if (rc != PMX_OK) return rc;
  if (N > 0) {
    invert_kernel<<<(unsigned)((N + 255) / 256), 256, 0, stream>>>(pos, N, order);
    PMX_LAUNCH_CHECK();
  }
  if (H == 0) return PMX_OK;
  const unsigned th = row_threads(H);
  if (H % 8 == 0 && aligned16(source) && aligned16(out)) {
    segment_rows_kernel<E, true><<<(unsigned)R, th, 0, stream>>>((const bf16_t*)source, order, offsets, H,
                                                             (bf16_t*)out);
  } else {
    segment_rows_kernel<E, false><<<(unsigned)R, th, 0, stream>>>((const bf16_t*)source, order, offsets, H,
                                                              (bf16_t*)out);
  }
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}

}  // namespace

extern "C" {

size_t pmx_segment_sum_workspace_bytes(int64_t num_src_rows, int64_t num_rows) {
  if (num_src_rows < 0 || num_rows <= 0 || num_rows > kRouteMaxSlots) return 0;
  const int64_t N = num_src_rows;
  size_t b = route_ws_bytes(N, (int32_t)num_rows);
  b = (b + 255) / 256 * 256;
  // phys, pos, order: int32 [N] each; counts [R], offsets [R+1]
  b += (size_t)(3 * N + 2 * num_rows + 1) * sizeof(int32_t) + 4 * 256;
  return b;
}

int pmx_moe_gather(const void* Y, const int32_t* pos, int64_t T, int32_t K, int64_t H, void* out,
                   pmx_stream_t stream) {
  return moe_gather_t<EltBF16>(Y, pos, T, K, H, out, stream);
}

int pmx_moe_gather_f16(const void* Y, const int32_t* pos, int64_t T, int32_t K, int64_t H, void* out,
                       pmx_stream_t stream) {
  return moe_gather_t<EltF16>(Y, pos, T, K, H, out, stream);
}

int pmx_combine_fwd(const void* Y, const int32_t* pos, const void* w, int64_t T, int32_t K, int64_t H,
                    void* out, pmx_stream_t stream) {
  return combine_fwd_t<EltBF16>(Y, pos, w, T, K, H, out, stream);
}

int pmx_combine_fwd_f16(const void* Y, const int32_t* pos, const void* w, int64_t T, int32_t K, int64_t H,
                        void* out, pmx_stream_t stream) {
  return combine_fwd_t<EltF16>(Y, pos, w, T, K, H, out, stream);
}

int pmx_combine_bwd_top1_rows(const void* dout, const void* Y, const int32_t* row_token, const void* w,
                              int64_t T, int64_t H, void* dY, void* dw, pmx_stream_t stream) {
  return combine_bwd_top1_rows_t<EltBF16>(dout, Y, row_token, w, T, H, dY, dw, stream);
}

int pmx_combine_bwd_top1_rows_f16(const void* dout, const void* Y, const int32_t* row_token, const void* w,
                                  int64_t T, int64_t H, void* dY, void* dw, pmx_stream_t stream) {
  return combine_bwd_top1_rows_t<EltF16>(dout, Y, row_token, w, T, H, dY, dw, stream);
}

int pmx_combine_bwd(const void* dout, const void* Y, const int32_t* pos, const void* w, int64_t T,
                    int32_t K, int64_t H, void* dY, void* dw, pmx_stream_t stream) {
  return combine_bwd_t<EltBF16>(dout, Y, pos, w, T, K, H, dY, dw, stream);
}

int pmx_combine_bwd_f16(const void* dout, const void* Y, const int32_t* pos, const void* w, int64_t T,
                        int32_t K, int64_t H, void* dY, void* dw, pmx_stream_t stream) {
  return combine_bwd_t<EltF16>(dout, Y, pos, w, T, K, H, dY, dw, stream);
}

int pmx_segment_sum(const void* source, const int64_t* index, int64_t N, int64_t H, int64_t num_rows,
                    void* out, void* workspace, size_t workspace_bytes, pmx_stream_t stream) {
  return segment_sum_t<EltBF16>(source, index, N, H, num_rows, out, workspace, workspace_bytes, stream);
}

int pmx_segment_sum_f16(const void* source, const int64_t* index, int64_t N, int64_t H, int64_t num_rows,
                        void* out, void* workspace, size_t workspace_bytes, pmx_stream_t stream) {
  return segment_sum_t<EltF16>(source, index, N, H, num_rows, out, workspace, workspace_bytes, stream);
}

}  // extern "C"
