// SwiGLU grouped GEMM for the PlaceMoE expert layer on gfx950.
//
// One persistent kernel template serves every GEMM of the layer:
//   KIND_FC1   X[a] @ [Wgate;Wup][g]^T with the SwiGLU forward epilogue
//   KIND_NT    A[a] @ B[g]^T                       (fc2 forward)
//   KIND_NN    A[a] @ B[g]                         (fc1 dgrad)
//   KIND_DG2   dY[a] @ Wdown[g] with the SwiGLU backward epilogue (fc2 dgrad)
//   KIND_TN    A[rows g]^T @ B[rows g]             (wgrad, ragged K)
// Groups are the per-copy row ranges [offsets[g], offsets[g+1]).  A fixed
// grid of blocks walks a tile list derived on the device from `offsets`, so
// empty groups cost nothing and the host never reads the counts.
//
// Tiles are 128x128x64, 256 threads = 4 waves in a 2x2 arrangement, each wave
// owning 64x64 of the output as 4x4 v_mfma_f32_16x16x32_bf16 tiles with fp32
// accumulators.  Operands are staged through double-buffered LDS with K
// contiguous per row (128-byte rows, 16-byte chunks XOR-swizzled by row so
// that both the MFMA fragment reads and the transposing stores are free of
// bank conflicts).  Operands that are N- or M-contiguous in HBM (dgrad
// weights, wgrad activations) are loaded as 4x8 blocks with 16-byte reads and
// transposed in registers on their way into LDS.

#include "common.h"

namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int NTHREADS = 256;
constexpr int kTileBytes = 128 * BK * 2;  // one operand tile in LDS
constexpr int kMaxGroups = 2048;

enum Kind { KIND_FC1 = 0, KIND_NT = 1, KIND_NN = 2, KIND_DG2 = 3, KIND_TN = 4 };

// Row-major bf16 operand whose rows may come from two tensors: rows below
// `split` from p0, the rest from p1 (row - split); per-group strides gs0/gs1.
struct RowSrc {
  const bf16_t* p0;
  const bf16_t* p1;
  int64_t gs0, gs1;
  int64_t ld;
  int64_t split;
};

struct GemmParams {
  RowSrc a, b;
  const int32_t* offsets;
  int32_t G;
  int64_t M, N, K;  // ragged-M kinds: N, K used.  KIND_TN: M, N used.
  int64_t I;        // SwiGLU width for KIND_FC1 / KIND_DG2
  bf16_t* c0;
  bf16_t* c1;
  int64_t ldc, cgs, csplit;
  bf16_t* gu;  // written by KIND_FC1, read by KIND_DG2
  bf16_t* act;
  bf16_t* dg1;
};

__device__ __forceinline__ const bf16_t* row_ptr(const RowSrc& s, int64_t g, int64_t row) {
  return row < s.split ? s.p0 + g * s.gs0 + row * s.ld : s.p1 + g * s.gs1 + (row - s.split) * s.ld;
}

__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * 128 + ((chunk ^ ((row ^ (row >> 3)) & 7)) << 4);
}

__device__ __forceinline__ uint4 ld16(const bf16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// Store a K-contiguous staging register set: thread t owns chunk (t & 7) of
// rows (t >> 3) + 32 i.
__device__ __forceinline__ void store_kc(char* lds, const uint4 (&r)[4], int t) {
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(lds + lds_off((t >> 3) + 32 * i, t & 7)) = r[i];
}

// Store a transposed staging set: r[j] holds 8 consecutive columns
// (c8 * 8 ..) of K-row k4 * 4 + j; LDS row = column, K contiguous.
__device__ __forceinline__ void store_kn(char* lds, const uint4 (&r)[4], int c8, int k4) {
  const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&r[0]);
  const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&r[1]);
  const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&r[2]);
  const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&r[3]);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int q = c >> 1;
    uint2 v;
    if (c & 1) {
      v.x = (w0[q] >> 16) | (w1[q] & 0xffff0000u);
      v.y = (w2[q] >> 16) | (w3[q] & 0xffff0000u);
    } else {
      v.x = (w0[q] & 0xffffu) | (w1[q] << 16);
      v.y = (w2[q] & 0xffffu) | (w3[q] << 16);
    }
    const int row = c8 * 8 + c;
    *reinterpret_cast<uint2*>(lds + lds_off(row, k4 >> 1) + (k4 & 1) * 8) = v;
  }
}

template <int KIND>
struct TileCtx {
  int64_t g;
  int64_t row0, row_end;  // ragged-M: output rows.  KIND_TN: reduction rows.
  int64_t mtile, ntile;
  int64_t nk;
};

// Global -> registers for K-tile kt.
template <int KIND>
__device__ __forceinline__ void load_tile(const GemmParams& P, const TileCtx<KIND>& tc, int64_t kt, int t,
                                          uint4 (&ra)[4], uint4 (&rb)[4]) {
  const uint4 zero = make_uint4(0, 0, 0, 0);
  const int64_t k0 = kt * BK;
  if constexpr (KIND == KIND_TN) {
    // Both operands are [row][m or n]; transposed staging.
    const int c8 = (t & 7) | ((t >> 7) << 3);
    const int k4 = (t >> 3) & 15;
    const int64_t m = tc.mtile * BM + c8 * 8;
    const int64_t n = tc.ntile * BN + c8 * 8;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t kk = k0 + k4 * 4 + j;
      const int64_t row = tc.row0 + kk;
      const bool kv = row < tc.row_end;
      ra[j] = (kv && m < P.M) ? ld16(P.a.p0 + row * P.a.ld + m) : zero;
      rb[j] = (kv && n < P.N) ? ld16(P.b.p0 + row * P.b.ld + n) : zero;
    }
  } else {
    // A: activation rows, K contiguous.
    const int kc = t & 7;
    const int64_t kcol = k0 + kc * 8;
    const bool kv = kcol < P.K;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = tc.row0 + (t >> 3) + 32 * i;
      ra[i] = (kv && row < tc.row_end) ? ld16(P.a.p0 + row * P.a.ld + kcol) : zero;
    }
    if constexpr (KIND == KIND_FC1) {
      const int64_t j0 = tc.ntile * 64;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = (t >> 3) + 32 * i;
        const int64_t j = j0 + (r >> 6) * 32 + (r & 31);
        const int64_t prow = ((r >> 5) & 1) ? P.I + j : j;
        rb[i] = (kv && j < P.I) ? ld16(row_ptr(P.b, tc.g, prow) + kcol) : zero;
      }
    } else if constexpr (KIND == KIND_NT) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t n = tc.ntile * BN + (t >> 3) + 32 * i;
        rb[i] = (kv && n < P.N) ? ld16(row_ptr(P.b, tc.g, n) + kcol) : zero;
      }
    } else {  // KIND_NN, KIND_DG2: B is [k][n], N contiguous; transposed staging.
      const int c8 = (t & 7) | ((t >> 7) << 3);
      const int k4 = (t >> 3) & 15;
      const int64_t n = tc.ntile * BN + c8 * 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t kk = k0 + k4 * 4 + j;
        rb[j] = (kk < P.K && n < P.N) ? ld16(row_ptr(P.b, tc.g, kk) + n) : zero;
      }
    }
  }
}

template <int KIND>
__device__ __forceinline__ void store_tile(char* As, char* Bs, int t, const uint4 (&ra)[4], const uint4 (&rb)[4]) {
  const int c8 = (t & 7) | ((t >> 7) << 3);
  const int k4 = (t >> 3) & 15;
  if constexpr (KIND == KIND_TN) {
    store_kn(As, ra, c8, k4);
    store_kn(Bs, rb, c8, k4);
  } else if constexpr (KIND == KIND_NN || KIND == KIND_DG2) {
    store_kc(As, ra, t);
    store_kn(Bs, rb, c8, k4);
  } else {
    store_kc(As, ra, t);
    store_kc(Bs, rb, t);
  }
}

__device__ __forceinline__ void mma_tile(const char* As, const char* Bs, int wm, int wn, int lane,
                                         f32x4_t (&acc)[4][4]) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    bf16x8_t a[4], b[4];
    const int chunk = ks * 4 + (lane >> 4);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      a[mt] = *reinterpret_cast<const bf16x8_t*>(As + lds_off(wm * 64 + mt * 16 + (lane & 15), chunk));
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
      b[nt] = *reinterpret_cast<const bf16x8_t*>(Bs + lds_off(wn * 64 + nt * 16 + (lane & 15), chunk));
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mt], b[nt], acc[mt][nt], 0, 0, 0);
  }
}

template <int KIND>
__device__ __forceinline__ void epilogue(const GemmParams& P, const TileCtx<KIND>& tc, int wm, int wn,
                                         int lane, const f32x4_t (&acc)[4][4]) {
  const int col_l = lane & 15;
  const int row_q = (lane >> 4) * 4;
  if constexpr (KIND == KIND_TN) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t m = tc.mtile * BM + wm * 64 + mt * 16 + row_q + j;
        if (m >= P.M) continue;
        bf16_t* crow = m < P.csplit ? P.c0 + tc.g * P.cgs + m * P.ldc : P.c1 + tc.g * P.cgs + (m - P.csplit) * P.ldc;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const int64_t n = tc.ntile * BN + wn * 64 + nt * 16 + col_l;
          if (n < P.N) crow[n] = (bf16_t)f32_to_bf16(acc[mt][nt][j]);
        }
      }
    }
  } else if constexpr (KIND == KIND_FC1) {
    const int64_t I = P.I;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t row = tc.row0 + wm * 64 + mt * 16 + row_q + j;
        if (row >= tc.row_end) continue;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int64_t col = tc.ntile * 64 + wn * 32 + nt * 16 + col_l;
          if (col >= I) continue;
          const float gb = round_bf16(acc[mt][nt][j]);
          const float ub = round_bf16(acc[mt][nt + 2][j]);
          const float s = round_bf16(silu_f32(gb));
          P.act[row * I + col] = (bf16_t)f32_to_bf16(s * ub);
          bf16_t* gurow = P.gu + row * 2 * I;
          gurow[col] = (bf16_t)f32_to_bf16(gb);
          gurow[I + col] = (bf16_t)f32_to_bf16(ub);
        }
      }
    }
  } else if constexpr (KIND == KIND_DG2) {
    const int64_t I = P.I;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t row = tc.row0 + wm * 64 + mt * 16 + row_q + j;
        if (row >= tc.row_end) continue;
        const bf16_t* gurow = P.gu + row * 2 * I;
        bf16_t* drow = P.dg1 + row * 2 * I;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const int64_t col = tc.ntile * BN + wn * 64 + nt * 16 + col_l;
          if (col >= I) continue;
          const float dact = round_bf16(acc[mt][nt][j]);
          const float g = bf16_to_f32(gurow[col]);
          const float u = bf16_to_f32(gurow[I + col]);
          const float s = round_bf16(silu_f32(g));
          const float d_silu = round_bf16(dact * u);
          const float sig = sigmoid_f32(g);
          drow[col] = (bf16_t)f32_to_bf16(d_silu * (sig * (1.0f + g * (1.0f - sig))));
          drow[I + col] = (bf16_t)f32_to_bf16(s * dact);
        }
      }
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t row = tc.row0 + wm * 64 + mt * 16 + row_q + j;
        if (row >= tc.row_end) continue;
        bf16_t* crow = P.c0 + row * P.ldc;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const int64_t col = tc.ntile * BN + wn * 64 + nt * 16 + col_l;
          if (col < P.N) crow[col] = (bf16_t)f32_to_bf16(acc[mt][nt][j]);
        }
      }
    }
  }
}

template <int KIND>
__global__ __launch_bounds__(NTHREADS, 2) void grouped_gemm_kernel(GemmParams P) {
  __shared__ __attribute__((aligned(16))) char lds[4 * kTileBytes];
  __shared__ int32_t tpre[kMaxGroups + 1];
  __shared__ int32_t scan_buf[NTHREADS];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int G = P.G;

  int64_t ntn, tiles_per_group = 0, total;
  if constexpr (KIND == KIND_TN) {
    const int64_t mtn = (P.M + BM - 1) / BM;
    ntn = (P.N + BN - 1) / BN;
    tiles_per_group = mtn * ntn;
    total = tiles_per_group * G;
  } else {
    ntn = (KIND == KIND_FC1) ? (P.I + 63) / 64 : (P.N + BN - 1) / BN;
    // Exclusive prefix of m-tiles per group: 8 groups per thread, then a
    // block scan of the 256 partial sums.
    int32_t loc[8];
    int32_t sum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int g = t * 8 + i;
      int32_t v = 0;
      if (g < G) v = (P.offsets[g + 1] - P.offsets[g] + BM - 1) / BM;
      loc[i] = sum;
      sum += v;
    }
    scan_buf[t] = sum;
    __syncthreads();
    for (int off = 1; off < NTHREADS; off <<= 1) {
      const int32_t add = t >= off ? scan_buf[t - off] : 0;
      __syncthreads();
      scan_buf[t] += add;
      __syncthreads();
    }
    const int32_t base = scan_buf[t] - sum;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int g = t * 8 + i;
      if (g < G) tpre[g] = base + loc[i];
    }
    if (t == NTHREADS - 1) tpre[G] = scan_buf[NTHREADS - 1];
    __syncthreads();
    total = (int64_t)tpre[G] * ntn;
  }

  // XCD-aware order: blocks are dispatched round-robin over the 8 XCDs, so
  // give the blocks of one XCD a contiguous run of each wave of tiles.
  const int64_t grid = gridDim.x;
  int64_t slot = blockIdx.x;
  if ((grid & 7) == 0) slot = (blockIdx.x & 7) * (grid >> 3) + (blockIdx.x >> 3);

  // Buffer b of the double buffer: A tile at lds + 2b*T, B tile right after.

  for (int64_t tile = slot; tile < total; tile += grid) {
    TileCtx<KIND> tc;
    if constexpr (KIND == KIND_TN) {
      tc.g = tile / tiles_per_group;
      const int64_t rem = tile - tc.g * tiles_per_group;
      tc.mtile = rem / ntn;
      tc.ntile = rem - tc.mtile * ntn;
      tc.row0 = P.offsets[tc.g];
      tc.row_end = P.offsets[tc.g + 1];
      tc.nk = (tc.row_end - tc.row0 + BK - 1) / BK;
    } else {
      const int64_t mt_global = tile / ntn;
      tc.ntile = tile - mt_global * ntn;
      int lo = 0, hi = G;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tpre[mid] <= mt_global) lo = mid;
        else hi = mid - 1;
      }
      tc.g = lo;
      tc.mtile = mt_global - tpre[lo];
      tc.row0 = P.offsets[lo] + tc.mtile * BM;
      tc.row_end = P.offsets[lo + 1];
      tc.nk = (P.K + BK - 1) / BK;
    }

    f32x4_t acc[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    if (tc.nk > 0) {
      uint4 ra[4], rb[4];
      load_tile<KIND>(P, tc, 0, t, ra, rb);
      store_tile<KIND>(lds, lds + kTileBytes, t, ra, rb);
      __syncthreads();
      for (int64_t kt = 0; kt < tc.nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < tc.nk;
        if (more) load_tile<KIND>(P, tc, kt + 1, t, ra, rb);
        char* cbuf = lds + cur * 2 * kTileBytes;
        char* nbuf = lds + (cur ^ 1) * 2 * kTileBytes;
        mma_tile(cbuf, cbuf + kTileBytes, wm, wn, lane, acc);
        if (more) store_tile<KIND>(nbuf, nbuf + kTileBytes, t, ra, rb);
        __syncthreads();
      }
    }
    epilogue<KIND>(P, tc, wm, wn, lane, acc);
  }
}

int g_num_cus = 0;

int grid_size() {
  if (g_num_cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -1;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
    g_num_cus = cus > 0 ? cus : 256;
  }
  return g_num_cus * 2;
}

template <int KIND>
int launch(const GemmParams& P, hipStream_t stream) {
  const int grid = grid_size();
  if (grid <= 0) return PMX_ERR_HIP;
  grouped_gemm_kernel<KIND><<<grid, NTHREADS, 0, stream>>>(P);
  PMX_LAUNCH_CHECK();
  return PMX_OK;
}

inline bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

RowSrc one(const void* p, int64_t gs, int64_t ld) {
  RowSrc s;
  s.p0 = s.p1 = static_cast<const bf16_t*>(p);
  s.gs0 = s.gs1 = gs;
  s.ld = ld;
  s.split = INT64_MAX;
  return s;
}

}  // namespace

extern "C" {

int pmx_gemm_fc1_swiglu_fwd(const void* X, const void* w_gate, const void* w_up, int64_t w_copy_stride,
                            const int32_t* offsets, int32_t G, int64_t A, int64_t H, int64_t I, void* gu,
                            void* act, pmx_stream_t stream) {
  if (G <= 0 || G > kMaxGroups || A < 0 || H <= 0 || I <= 0) return PMX_ERR_ARG;
  if (H % 8 || I % 8) return PMX_ERR_SHAPE;
  if (A == 0) return PMX_OK;
  if (!X || !w_gate || !w_up || !offsets || !gu || !act) return PMX_ERR_ARG;
  if (!a16(X) || !a16(w_gate) || !a16(w_up)) return PMX_ERR_SHAPE;
  GemmParams P = {};
  P.a = one(X, 0, H);
  P.b.p0 = static_cast<const bf16_t*>(w_gate);
  P.b.p1 = static_cast<const bf16_t*>(w_up);
  P.b.gs0 = P.b.gs1 = w_copy_stride;
  P.b.ld = H;
  P.b.split = I;
  P.offsets = offsets;
  P.G = G;
  P.K = H;
  P.N = 2 * I;
  P.I = I;
  P.gu = static_cast<bf16_t*>(gu);
  P.act = static_cast<bf16_t*>(act);
  return launch<KIND_FC1>(P, stream);
}

int pmx_group_gemm_nt(const void* A, const void* B, const int32_t* offsets, int32_t G, int64_t M, int64_t N,
                      int64_t K, void* C, pmx_stream_t stream) {
  if (G <= 0 || G > kMaxGroups || M < 0 || N <= 0 || K <= 0) return PMX_ERR_ARG;
  if (N % 8 || K % 8) return PMX_ERR_SHAPE;
  if (M == 0) return PMX_OK;
  if (!A || !B || !offsets || !C) return PMX_ERR_ARG;
  if (!a16(A) || !a16(B)) return PMX_ERR_SHAPE;
  GemmParams P = {};
  P.a = one(A, 0, K);
  P.b = one(B, N * K, K);
  P.offsets = offsets;
  P.G = G;
  P.N = N;
  P.K = K;
  P.c0 = static_cast<bf16_t*>(C);
  P.ldc = N;
  return launch<KIND_NT>(P, stream);
}

int pmx_group_gemm_nn(const void* A, const void* B0, const void* B1, int64_t b_copy_stride, int64_t b_split,
                      const int32_t* offsets, int32_t G, int64_t M, int64_t N, int64_t K, void* C,
                      pmx_stream_t stream) {
  if (G <= 0 || G > kMaxGroups || M < 0 || N <= 0 || K <= 0) return PMX_ERR_ARG;
  if (N % 8 || K % 8) return PMX_ERR_SHAPE;
  if (M == 0) return PMX_OK;
  if (!A || !B0 || !offsets || !C) return PMX_ERR_ARG;
  if (!a16(A) || !a16(B0) || (B1 && !a16(B1))) return PMX_ERR_SHAPE;
  GemmParams P = {};
  P.a = one(A, 0, K);
  P.b = one(B0, b_copy_stride, N);
  if (B1 != nullptr) {
    if (b_split <= 0 || b_split >= K) return PMX_ERR_ARG;
    P.b.p1 = static_cast<const bf16_t*>(B1);
    P.b.split = b_split;
  }
  P.offsets = offsets;
  P.G = G;
  P.N = N;
  P.K = K;
  P.c0 = static_cast<bf16_t*>(C);
  P.ldc = N;
  return launch<KIND_NN>(P, stream);
}

int pmx_gemm_fc2_dgrad_swiglu_bwd(const void* dY, const void* w_down, const void* gu, const int32_t* offsets,
                                  int32_t G, int64_t A, int64_t H, int64_t I, void* dG1, pmx_stream_t stream) {
  if (G <= 0 || G > kMaxGroups || A < 0 || H <= 0 || I <= 0) return PMX_ERR_ARG;
  if (H % 8 || I % 8) return PMX_ERR_SHAPE;
  if (A == 0) return PMX_OK;
  if (!dY || !w_down || !gu || !offsets || !dG1) return PMX_ERR_ARG;
  if (!a16(dY) || !a16(w_down)) return PMX_ERR_SHAPE;
  GemmParams P = {};
  P.a = one(dY, 0, H);
  P.b = one(w_down, H * I, I);
  P.offsets = offsets;
  P.G = G;
  P.N = I;
  P.K = H;
  P.I = I;
  P.gu = static_cast<bf16_t*>(const_cast<void*>(gu));
  P.dg1 = static_cast<bf16_t*>(dG1);
  return launch<KIND_DG2>(P, stream);
}

int pmx_group_gemm_tn(const void* A, const void* B, const int32_t* offsets, int32_t G, int64_t M, int64_t N,
                      void* C0, void* C1, int64_t c_copy_stride, int64_t c_split, pmx_stream_t stream) {
  if (G <= 0 || G > kMaxGroups || M <= 0 || N <= 0) return PMX_ERR_ARG;
  if (M % 8 || N % 8) return PMX_ERR_SHAPE;
  if (!A || !B || !offsets || !C0) return PMX_ERR_ARG;
  if (!a16(A) || !a16(B)) return PMX_ERR_SHAPE;
  GemmParams P = {};
  P.a = one(A, 0, M);
  P.b = one(B, 0, N);
  P.offsets = offsets;
  P.G = G;
  P.M = M;
  P.N = N;
  P.c0 = static_cast<bf16_t*>(C0);
  P.c1 = C1 ? static_cast<bf16_t*>(C1) : static_cast<bf16_t*>(C0);
  P.cgs = c_copy_stride;
  P.ldc = N;
  P.csplit = C1 ? c_split : INT64_MAX;
  if (C1 && (c_split <= 0 || c_split >= M)) return PMX_ERR_ARG;
  return launch<KIND_TN>(P, stream);
}

}  // extern "C"
