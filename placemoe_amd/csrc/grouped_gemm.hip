// SwiGLU grouped GEMM for the PlaceMoE expert layer on gfx950.
//
// One persistent kernel template serves every GEMM of the layer:
//   KIND_FC1   X[a] @ [Wgate;Wup][g]^T with the SwiGLU forward epilogue
//   KIND_NT    A[a] @ B[g]^T                       (fc2 forward)
//   KIND_NN    A[a] @ B[g]                         (fc1 dgrad)
//   KIND_NNS   A[a] @ B[g] with the SwiGLU backward epilogue (fc2 dgrad)
//   KIND_TN    A[rows g]^T @ B[rows g]             (wgrad, ragged K)
// Groups are the per-copy row ranges [offsets[g], offsets[g+1]).  A grid of
// one block per CU walks a tile list derived on the device from `offsets`,
// so empty groups cost nothing and the host never reads the counts.
//
// Block tile 256 x 256, K in steps of 64; 8 waves (two per SIMD) in a 2 x 4
// arrangement, each owning 128 x 64 of the output as 4 x 2 tiles of
// v_mfma_f32_32x32x16_bf16 with fp32 accumulators: while one wave of a SIMD
// waits for LDS, a load or the barrier, the other keeps the matrix core busy.
//
// Operands stream HBM -> LDS through two 64 KB stages, either with
// buffer_load ... lds (no VGPR staging) or, in the register-staged variant,
// through one VGPR per 1 KB piece: K-tile p+1 lands in one stage while
// K-tile p is multiplied from the other.  64-deep K-tiles make every row segment a load
// instruction fetches one whole 128-byte line.  A block walks its tiles as one
// stream of K-tiles, so the next tile's first loads overlap the current
// tile's end and epilogue.  The loads are issued as inline asm, one every
// other pinned MFMA group of the first two k-steps (one per group of the
// first k-step for the wgrad), and waited for by hand (vmcnt).  Rows or columns outside a group, outside N/M, or past K are
// masked by buffer range checks (an out-of-range offset loads zeros).
//
// LDS layouts, both XOR-swizzled in 16-byte chunks so that the fragment reads
// are free of bank conflicts:
//   K-contiguous operands (activation rows, fc1/fc2 weights): [row][64 k],
//     128-byte rows, chunk c stored at c ^ ((row >> 1) & 7); fragments
//     are ds_read_b128.
//   M/N-contiguous operands (dgrad weights, both wgrad operands): [64 k][W],
//     chunk c of k-row kk stored at c ^ 4*(kk & 3); fragments are pairs of
//     ds_read_b64_tr_b16, which transpose 4x16 blocks on the way out of LDS.

#include "common.h"
#include "ktile.h"

// Element type of this build of the file: bf16, or fp16 with -DPMX_ELT_F16
// (the C-ABI entry points then carry the suffix _f16).  Both builds share
// every kernel; only the MFMA instruction and the fp32 conversions differ.
#ifdef PMX_ELT_F16
#define PMX_GEMM_FN(name) name##_f16
#else
#define PMX_GEMM_FN(name) name
#endif

namespace {

#ifdef PMX_ELT_F16
using Elt = EltF16;
#else
using Elt = EltBF16;
#endif

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// The MFMAs of the element type; fragments hold the 16-bit patterns as
// bf16x8_t either way (the LDS reads move bits).
__device__ __forceinline__ f32x16_t mfma32(const bf16x8_t& b, const bf16x8_t& a, const f32x16_t& c) {
#ifdef PMX_ELT_F16
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, b), __builtin_bit_cast(f16x8_t, a), c, 0,
                                                 0, 0);
#else
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, c, 0, 0, 0);
#endif
}
__device__ __forceinline__ f32x4_t mfma16(const bf16x8_t& b, const bf16x8_t& a, const f32x4_t& c) {
#ifdef PMX_ELT_F16
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, b), __builtin_bit_cast(f16x8_t, a), c, 0,
                                                 0, 0);
#else
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(b, a, c, 0, 0, 0);
#endif
}

// K-tiles are 64 deep so that every K-contiguous row segment a load
// instruction fetches is one whole 128-byte line: with 32-deep K-tiles each
// segment is half a line, the L1 issues twice the requests to L2 for the
// same bytes and the texture unit backs up behind it.
constexpr int BN = 256, BK = 64;
// Two pipeline stages of (BM + BN) x 64 bf16 (64 KB each) next to the group
// prefix and the block's decoded tile table in 160 KB of LDS; the epilogue
// stages its output in the stage just freed.
constexpr int NSTAGE = 2;
// Eight waves, two per SIMD, in a 2 x 4 arrangement: each owns 128 x 64 of
// the output as 4 x 2 tiles of v_mfma_f32_32x32x16_bf16 (128 AGPRs), so that
// while one wave of a SIMD waits (for LDS, a load or the barrier) the other
// keeps the matrix core busy.
constexpr int NWAVES = 8, WAVES_N = 4;
constexpr int NTHREADS = 64 * NWAVES;
constexpr int WROWS = 128, WCOLS = 64;  // output tile of one wave
constexpr int MT = WROWS / 32, NTT = WCOLS / 32;
constexpr int kMaxGroups = 2048;
// Decoded tiles per block kept in LDS; a block's tiles past the table are
// decoded on the spot.  PMX_TILE_TAB overrides it for a test build that runs
// that path at small shapes.
#ifndef PMX_TILE_TAB
#define PMX_TILE_TAB 1024
#endif
constexpr int kTileTab = PMX_TILE_TAB;
static_assert(kTileTab >= 1 && kTileTab <= 1024, "tile table: 1 .. 1024 entries (16 KB of LDS)");
// A table entry packs the group id in 12 bits and the n-tile above it.
static_assert(kMaxGroups <= (1 << 12), "group ids must fit the tile table's 12 bits");
constexpr uint32_t kOOB = 0x80000000u;  // buffer offset that always fails the range check
constexpr uint32_t kRsrcWord3 = 0x00020000u;

enum Kind { KIND_FC1 = 0, KIND_NT = 1, KIND_NN = 2, KIND_NNS = 3, KIND_TN = 4 };

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))
#define LDS_TR_PTR(p) ((__attribute__((address_space(3))) bf16x4_t*)(p))

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
  int64_t M, N, K;  // ragged-M kinds: N, K used.  KIND_TN: M, N, and K = rows of A and B.
  int64_t I;        // SwiGLU width for KIND_FC1 and KIND_NNS
  bf16_t* c0;
  bf16_t* c1;
  int64_t ldc, cgs, csplit;
  bf16_t* gu;  // written by KIND_FC1
  bf16_t* act;
  const bf16_t* gin;  // KIND_NNS: the forward's gate/up rows [A, 2I]
  // Top-1 row map (KIND_NN, KIND_NT; null: none).  KIND_NN writes output row
  // r to row row_tok[r] of c0 instead of row r.  KIND_NT writes row r to c0
  // and also cout[row_tok[r]] = bf16(0 + bf16(row * row_w[r])).
  const int32_t* row_tok;
  const bf16_t* row_w;
  bf16_t* cout;
};

template <int KIND>
constexpr bool a_is_mn() { return KIND == KIND_TN; }
template <int KIND>
constexpr bool b_is_mn() { return KIND == KIND_NN || KIND == KIND_NNS || KIND == KIND_TN; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0x7fffffffull ? 0x7fffffffu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, (int)kRsrcWord3);
}

// 16-byte chunk swizzle of the 128-byte rows of K-contiguous tiles: 16
// consecutive rows read at one logical chunk hit 16 distinct (row parity,
// chunk) bank groups.
__device__ __forceinline__ int kc_swz(int row) { return (row >> 1) & 7; }

// Per-tile operand description.  Each DMA instruction of this wave has a
// tile-invariant per-lane byte offset `voff[q0]` (kOOB where the lane's chunk
// lies outside the operand); the K-tile advance goes into the scalar offset.
// Operands whose K is not a multiple of 64 mask, in their last K-tile, the
// lanes whose bit in `tmask` is clear (their chunk or k-row lies past K).
//
// Per K-tile a wave only adds to the scalar offset (and, for wgrad operands,
// rebases one descriptor): every per-tile quantity is set up once per tile.
struct Operand {
  __amdgpu_buffer_rsrc_t r0, r1;  // K-contiguous: r1 holds fc1's up rows;
                                  // MN weights: k-rows below / from `split`
  const char* base;               // wgrad operands: the group's first row ...
  uint64_t bytes;                 // ... and the bytes of its rows (descriptor rebased per K-tile)
  __amdgpu_buffer_rsrc_t rk;      // wgrad operands: descriptor of the K-tile being issued
  uint32_t ldb;                   // bytes between consecutive (k-)rows
  int32_t split;                  // MN weights: first k-row taken from r1
  uint32_t split_bytes;           // split * ldb
  int32_t ktail;                  // the partial last K-tile, -1 if none
  uint32_t voff[4];
  uint32_t tmask;                 // bit q0: instruction q0's lane lies within K in K-tile ktail
};

// The per-lane offset of instruction q0, masked past K in the tail K-tile.
__device__ __forceinline__ uint32_t lane_off(const Operand& op, int q0, bool tail) {
  return (tail && !((op.tmask >> q0) & 1u)) ? kOOB : op.voff[q0];
}

// Where one output tile lies: group, m/n tile, its rows (ragged kinds: the
// tile's first row and the group's end), and its K-tile count.
struct TileInfo {
  int32_t g, mtile, ntile, row0, row_end, nk;
};

template <int KIND, int BM>
struct Tile {
  TileInfo i;
  Operand A, B;
};

// Wave-uniform copies (SGPRs) of values every lane holds alike: tile
// bookkeeping read from LDS or memory would otherwise stay in VGPRs, and
// descriptor selections on it would become branches around each load.
__device__ __forceinline__ int32_t uni(int32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uni64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// One buffer->LDS instruction: 64 lanes x 16 bytes land contiguously at `dst`
// (M0 holds the wave's LDS address).  Written as inline asm so that the
// compiler does not track it: its own LDS-DMA bookkeeping cannot tell the
// pipeline stages apart and would wait for younger stages before every LDS
// read.  Completion is tracked by hand (wait_loads) and published to the
// other waves by block_barrier, both of which clobber memory; this asm does
// not, so LDS reads of other stages may be scheduled across it.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, char* dst, uint32_t voff, uint32_t soff) {
  const uint32_t m0 = (uint32_t)(uintptr_t)LDS_PTR(dst);
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(m0));
}

// An empty descriptor: every offset fails its range check and loads zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t empty_rsrc(const void* base) { return make_rsrc(base, 0); }

// Per wave, the buffer->LDS instructions that bring in an R-row (or R-wide)
// operand tile of one K-tile: R x 64 bf16 in 1 KB instructions.
template <int R>
constexpr int loads_per_wave() { return R * BK * 2 / 1024 / NWAVES; }

// K-contiguous operand, R rows x 64 k: instruction q = q0*NWAVES + wave
// covers 8 rows x 128 bytes.  Lane i of instruction q fills row 8q + i/8,
// physical chunk i%8, i.e. logical chunk (i%8) ^ swz(row).
// FC1's virtual B rows alternate 32 gate rows and 32 up rows; a wave's
// instructions all read one of the two (setup_operands puts it in r0).
// FAST (K a multiple of 64): no K tail to mask, and `live` is not read: a
// finished issue cursor keeps its last tile with kt = 0, so its pipeline
// slots re-load that tile's first K-tile (in bounds; never multiplied).
template <int R, bool SPLIT_ROWS, int Q0B = 0, int Q0E = loads_per_wave<R>(), bool FAST = false>
__device__ __forceinline__ void dma_kc(char* lds, const Operand& op, int32_t kt, bool live, int wave) {
  if constexpr (FAST) {
    const uint32_t soff = (uint32_t)kt * (BK * 2);
#pragma unroll
    for (int q0 = Q0B; q0 < Q0E; ++q0) {
      const int q = q0 * NWAVES + wave;
      dma16(op.r0, lds + q * 1024, op.voff[q0], soff);
    }
    return;
  }
  const uint32_t soff = live ? (uint32_t)kt * (BK * 2) : 0u;
  const bool tail = kt == op.ktail;
  const __amdgpu_buffer_rsrc_t none = empty_rsrc(op.base);
  const __amdgpu_buffer_rsrc_t r0 = live ? op.r0 : none;
#pragma unroll
  for (int q0 = Q0B; q0 < Q0E; ++q0) {
    const int q = q0 * NWAVES + wave;
    dma16(r0, lds + q * 1024, lane_off(op, q0, tail), soff);
  }
}

// M/N-contiguous operand, 64 k-rows x W columns: instruction q = q0*NWAVES
// + wave covers 512/W k-rows x 2W bytes.  Lane i of instruction q fills
// k-row q*ROWS + i/CH, physical chunk i%CH = logical chunk ^ 4*(kk&3).
// REBASE (wgrad): the descriptor starts at the K-tile's first row and ends
// with the group, so rows past the group load zeros.  Otherwise (dgrad
// weights) the K-tile advance is a scalar offset into r0 (k-rows below split)
// or r1, and the lanes past K are masked in the last K-tile.
// FAST (dgrad weights with K a multiple of 64 and no split): every k-row
// comes from r0, no K tail, no `live` test (see dma_kc).
template <int W, bool REBASE, int Q0B = 0, int Q0E = loads_per_wave<W>(), bool FAST = false>
__device__ __forceinline__ void dma_mn(char* lds, const Operand& op, int32_t kt, bool live, int wave) {
  constexpr int ROWS = 1024 / (2 * W);
  if constexpr (FAST && REBASE) {
    // Weight gradient whose operands fit 31-bit offsets: one descriptor per
    // group, the K-tile advance in the scalar offset; the range check covers
    // vector plus scalar offset, so rows past the group's end load zeros
    // (pinned by a GPU test with NaN rows past the last group).
    const uint32_t soff = (uint32_t)kt * (uint32_t)BK * op.ldb;
#pragma unroll
    for (int q0 = Q0B; q0 < Q0E; ++q0) {
      const int q = q0 * NWAVES + wave;
      dma16(op.r0, lds + q * 1024, op.voff[q0], soff);
    }
  } else if constexpr (FAST && !REBASE) {
#pragma unroll
    for (int q0 = Q0B; q0 < Q0E; ++q0) {
      const int q = q0 * NWAVES + wave;
      const uint32_t k = (uint32_t)kt * BK + (uint32_t)(q * ROWS);  // first k-row of the instruction
      dma16(op.r0, lds + q * 1024, op.voff[q0], k * op.ldb);
    }
  } else if constexpr (REBASE) {
    // op.rk is the window of the K-tile being issued (rebase_ktile), kept up
    // to date by the issue cursor.
#pragma unroll
    for (int q0 = Q0B; q0 < Q0E; ++q0) {
      const int q = q0 * NWAVES + wave;
      dma16(op.rk, lds + q * 1024, op.voff[q0], 0u);
    }
  } else {
    const bool tail = kt == op.ktail;
    const __amdgpu_buffer_rsrc_t none = empty_rsrc(op.base);
#pragma unroll
    for (int q0 = Q0B; q0 < Q0E; ++q0) {
      const int q = q0 * NWAVES + wave;
      const int32_t k = kt * BK + q * ROWS;  // first k-row of the instruction
      const bool second = k >= op.split;
      const uint32_t soff = live ? (uint32_t)k * op.ldb - (second ? op.split_bytes : 0u) : 0u;
      dma16(!live ? none : second ? op.r1 : op.r0, lds + q * 1024, lane_off(op, q0, tail), soff);
    }
  }
}

// Point a weight-gradient operand's descriptor at K-tile kt of its group:
// the window starts at the K-tile's first row and ends with the group, in
// 64-bit arithmetic (ktile.h).  `live` false: an empty window (loads zeros).
__device__ __forceinline__ void rebase_ktile(Operand& op, int32_t kt, bool live) {
  const pmx::KTileWindow win = pmx::ktile_window(op.bytes, op.ldb, kt, live);
  const uint64_t base = reinterpret_cast<uint64_t>(op.base) + win.offset;
  op.rk = make_rsrc(reinterpret_cast<const void*>(uni64((int64_t)base)), (uint64_t)uni64((int64_t)win.bytes));
}

// Issue this wave's share of K-tile kt of a tile into `stage`.  `live` is
// false for the pipeline slots past the block's last tile: they go through an
// empty descriptor, so every step issues the same number of loads.
// PART selects the operands: 0 = A, 1 = B, 2 = both.
template <int KIND, int BM, bool FAST, int PART = 2>
__device__ __forceinline__ void issue_stage(char* stage, const Tile<KIND, BM>& tc, int32_t kt, bool live, int wave) {
  char* As = stage;
  char* Bs = stage + BM * BK * 2;
  if constexpr (PART != 1) {
    if constexpr (a_is_mn<KIND>()) dma_mn<BM, true, 0, loads_per_wave<BM>(), FAST>(As, tc.A, kt, live, wave);
    else dma_kc<BM, false, 0, loads_per_wave<BM>(), FAST>(As, tc.A, kt, live, wave);
  }
  if constexpr (PART != 0) {
    if constexpr (b_is_mn<KIND>()) dma_mn<BN, KIND == KIND_TN, 0, loads_per_wave<BN>(), FAST>(Bs, tc.B, kt, live, wave);
    else dma_kc<BN, KIND == KIND_FC1, 0, loads_per_wave<BN>(), FAST>(Bs, tc.B, kt, live, wave);
  }
}

// Instruction Q0 of this wave's share of operand OPER (0 = A, 1 = B).
template <int KIND, int BM, bool FAST, int OPER, int Q0>
__device__ __forceinline__ void issue_one(char* stage, const Tile<KIND, BM>& tc, int32_t kt, bool live, int wave) {
  if constexpr (OPER == 0) {
    if constexpr (a_is_mn<KIND>()) dma_mn<BM, true, Q0, Q0 + 1, FAST>(stage, tc.A, kt, live, wave);
    else dma_kc<BM, false, Q0, Q0 + 1, FAST>(stage, tc.A, kt, live, wave);
  } else {
    char* Bs = stage + BM * BK * 2;
    if constexpr (b_is_mn<KIND>()) dma_mn<BN, KIND == KIND_TN, Q0, Q0 + 1, FAST>(Bs, tc.B, kt, live, wave);
    else dma_kc<BN, KIND == KIND_FC1, Q0, Q0 + 1, FAST>(Bs, tc.B, kt, live, wave);
  }
}


// RS: piece Q0 (A pieces 0 .. QA-1, then B) of this wave's share of K-tile
// kt, loaded into a register with the addressing of the buffer->LDS
// instruction it replaces (FAST ragged-M kinds), and its store to the LDS
// position that instruction fills.
template <int KIND, int BM, int PIECE>
__device__ __forceinline__ uint4 load_piece(const Tile<KIND, BM>& tc, int32_t kt, int wave) {
  constexpr int QA = loads_per_wave<BM>();
  if constexpr (PIECE < QA) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(tc.A.r0, tc.A.voff[PIECE],
                                                                          (uint32_t)kt * (BK * 2), 0));
  } else {
    constexpr int Q0 = PIECE - QA;
    uint32_t soff;
    if constexpr (b_is_mn<KIND>()) {
      constexpr int ROWS = 1024 / (2 * BN);
      soff = ((uint32_t)kt * BK + (uint32_t)((Q0 * NWAVES + wave) * ROWS)) * tc.B.ldb;
    } else {
      soff = (uint32_t)kt * (BK * 2);
    }
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(tc.B.r0, tc.B.voff[Q0], soff, 0));
  }
}
template <int BM, int PIECE>
__device__ __forceinline__ void store_piece(char* stage, int wave, int lane, const uint4& v) {
  constexpr int QA = loads_per_wave<BM>();
  char* base = PIECE < QA ? stage : stage + BM * BK * 2;
  constexpr int Q0 = PIECE < QA ? PIECE : PIECE - QA;
  *reinterpret_cast<uint4*>(base + (Q0 * NWAVES + wave) * 1024 + lane * 16) = v;
}

// Fragment of a K-contiguous tile: lane l holds row (rb + l%32), k = ks*16 + (l/32)*8 + 0..7.
__device__ __forceinline__ bf16x8_t frag_kc(const char* t, int rb, int ks, int lane) {
  const int row = rb + (lane & 31);
  const int chunk = ks * 2 + (lane >> 5);
  return *reinterpret_cast<const bf16x8_t*>(t + row * (BK * 2) + ((chunk ^ kc_swz(row)) << 4));
}

// Fragment of an M/N-contiguous tile (W columns): lane l holds column
// cb + l%32 at k = ks*16 + (l/32)*8 + 0..7, built from two transposing reads.
// Within each 16-lane group, lane i addresses row i/4 and columns 4*(i%4)..+3
// of a 4x16 block and receives column i of that block.
template <int W>
__device__ __forceinline__ bf16x8_t frag_mn(const char* t, int cb, int ks, int lane) {
  const int gq = lane >> 4, i = lane & 15;
  const int col = cb + 16 * (gq & 1) + (i & 3) * 4;
  const int c = col >> 3, half = (col >> 2) & 1;
  bf16x4_t v[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int kk = ks * 16 + (gq >> 1) * 8 + h * 4 + (i >> 2);
    const char* p = t + kk * (2 * W) + ((c ^ (4 * (kk & 3))) << 4) + half * 8;
    v[h] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_TR_PTR(p));
  }
  return bf16x8_t{v[0][0], v[0][1], v[0][2], v[0][3], v[1][0], v[1][1], v[1][2], v[1][3]};
}

// The wave's operand fragments of one 16-deep k-step of a stage.
template <int BM>
struct Frags {
  bf16x8_t a[MT], b[NTT];
};

template <int KIND, int BM>
__device__ __forceinline__ void read_frags(const char* stage, int ks, int wm, int wn, int lane, Frags<BM>& f) {
  const char* As = stage;
  const char* Bs = stage + BM * BK * 2;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int rb = wm * WROWS + mt * 32;
    if constexpr (a_is_mn<KIND>()) f.a[mt] = frag_mn<BM>(As, rb, ks, lane);
    else f.a[mt] = frag_kc(As, rb, ks, lane);
  }
#pragma unroll
  for (int nt = 0; nt < NTT; ++nt) {
    const int cb = wn * WCOLS + nt * 32;
    if constexpr (b_is_mn<KIND>()) f.b[nt] = frag_mn<BN>(Bs, cb, ks, lane);
    else f.b[nt] = frag_kc(Bs, cb, ks, lane);
  }
}

// Fragment J of a k-step: A fragments 0 .. MT-1, then B fragments 0 .. NTT-1.
template <int KIND, int BM, int J>
__device__ __forceinline__ void read_frag(const char* stage, int ks, int wm, int wn, int lane, Frags<BM>& f) {
  if constexpr (J < MT) {
    const int rb = wm * WROWS + J * 32;
    if constexpr (a_is_mn<KIND>()) f.a[J] = frag_mn<BM>(stage, rb, ks, lane);
    else f.a[J] = frag_kc(stage, rb, ks, lane);
  } else {
    const char* Bs = stage + BM * BK * 2;
    const int cb = wn * WCOLS + (J - MT) * 32;
    if constexpr (b_is_mn<KIND>()) f.b[J - MT] = frag_mn<BN>(Bs, cb, ks, lane);
    else f.b[J - MT] = frag_kc(Bs, cb, ks, lane);
  }
}

// The I-th fragment read of a k-step, in the order the MFMAs (mt-major)
// consume them: A0, B0 .. B(NTT-1), then A1 .. A(MT-1).  Fragment ids as in
// read_frag: A fragments 0 .. MT-1, B fragments MT .. MT+NTT-1.
constexpr int frag_order(int i) { return i == 0 ? 0 : i <= NTT ? MT + i - 1 : i - NTT; }

// MFMAs I .. I+N-1 of a k-step (index mt * NTT + nt).  FIRST: the tile's
// first k-step, whose MFMAs start from zero (an inline-constant accumulator
// operand) instead of from cleared registers.
template <int BM, int I, int N, bool FIRST = false>
__device__ __forceinline__ void mma_some(const Frags<BM>& f, f32x16_t (&acc)[MT][NTT]) {
#pragma unroll
  for (int x = I; x < I + N; ++x)
    acc[x / NTT][x % NTT] = mfma32(f.b[x % NTT], f.a[x / NTT], FIRST ? f32x16_t{} : acc[x / NTT][x % NTT]);
}

template <int BM>
__device__ __forceinline__ void mma_frags(const Frags<BM>& f, f32x16_t (&acc)[MT][NTT]) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTT; ++nt)
      acc[mt][nt] = mfma32(f.b[nt], f.a[mt], acc[mt][nt]);
}

// Compile-time loop: f(Int<I>{}) for I = B .. E-1, so that accumulator
// indices stay constants however large the unrolled body grows.
template <int V>
struct Int {
  static constexpr int value = V;
};
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(Int<B>{});
    static_for<B + 1, E>(f);
  }
}

// The MFMAs take the B fragment as their first operand, so each accumulator
// holds its 32 x 32 output tile transposed: element i of acc[mt][nt] in lane
// l is output row l%32, column 8*(i/4) + 4*(l/32) + i%4.  A lane therefore
// holds runs of 4 consecutive columns of one row, which go to LDS as single
// 8-byte writes.
//
// Epilogue: the wave's 128 x 64 output tile passes through LDS as bf16 in two
// rounds of 64 rows (8 KB), then leaves as 16-byte row segments, eight rows of
// 128 bytes per store instruction.  The stores are streaming (non-temporal):
// outputs of hundreds of MB are not read back by this kernel, and keeping them
// out of the L2 leaves it to the operand strips (measured: Qwen3-shape fc2
// 797 -> 830 TFLOP/s, layer 4.84 -> 4.77 ms; DeepSeek-V3 shape +0.4%).  The staging area is the wave's own share
// of the stage just freed: the eight 1 KB chunks k*NWAVES + wave that its
// buffer->LDS loads fill, so no other wave reads or writes them until this
// wave issues its next loads.  Rows of a round are 128 bytes; 16-byte chunk c
// of row r sits at c ^ ((r >> 1) & 7).

__device__ __forceinline__ uint2 pack4(float a, float b, float c, float d) { return make_uint2(Elt::pack2(a, b), Elt::pack2(c, d)); }
__device__ __forceinline__ uint2 acc4(const f32x16_t& a, int i) { return pack4(a[i], a[i + 1], a[i + 2], a[i + 3]); }

// Byte offset, inside the stage, of byte `x` of row r (0..63) of the wave's staging area.
__device__ __forceinline__ int epi_off(int wave, int r, int x) {
  const int chunk = (x >> 4) ^ ((r >> 1) & 7);
  return ((r >> 3) * NWAVES + wave) * 1024 + (r & 7) * 128 + (chunk << 4) + (x & 15);
}

// Stage rows 64*half .. +63 of the wave's tile (columns 0 .. 32*NC-1 of the
// wave's 64) from `v(mt, nt, i)`: elements i .. i+3 of acc[mt][nt] as four bf16.
template <int NC, typename F>
__device__ __forceinline__ void stage_half(char* stage, int wave, int lane, int half, F v) {
  const int rl = lane & 31, h = lane >> 5;
#pragma unroll
  for (int mtl = 0; mtl < 2; ++mtl)
#pragma unroll
    for (int nt = 0; nt < NC; ++nt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int mt = 2 * half + mtl;
        const int r = mtl * 32 + rl;
        const int col = nt * 32 + 8 * j + 4 * h;
        *reinterpret_cast<uint2*>(stage + epi_off(wave, r, col * 2)) = v(mt, nt, 4 * j);
      }
}

__device__ __forceinline__ uint4 staged_chunk(const char* stage, int wave, int r, int chunk) {
  return *reinterpret_cast<const uint4*>(stage + epi_off(wave, r, chunk * 16));
}

// Rows row0 .. row0+63 of a row-major bf16 tensor of `ld` elements per row
// (one epilogue round) as a buffer descriptor that ends at row `row_end`, so
// that the range check drops the loads (zeros) and stores of rows past the
// tile's group: no 64-bit address arithmetic and no branch per store.  The
// whole offset, row and column, is the 32-bit vector offset (kOOB for columns
// past the tensor).  (The range check covers the sum of the vector and scalar
// offsets, which the weight gradient's FAST loads rely on; the stores keep
// the scalar offset at 0.)
struct OutWin {
  __amdgpu_buffer_rsrc_t r;
  uint32_t rowb;  // bytes per row
};
__device__ __forceinline__ OutWin out_window(const bf16_t* base, int64_t row0, int64_t row_end, int64_t ld) {
  const int64_t rows = row_end - row0 < 0 ? 0 : (row_end - row0 > 64 ? 64 : row_end - row0);
  return {make_rsrc(base + row0 * ld, (uint64_t)(rows * ld * 2)), (uint32_t)(ld * 2)};
}
constexpr int kCpolNT = 2;  // buffer instruction cache policy: non-temporal (streaming)
// Row `row` further on from a lane's offset `voff`.
__device__ __forceinline__ void win_store(const OutWin& w, uint32_t voff, uint32_t row, const uint4& v) {
  __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{v.x, v.y, v.z, v.w}, w.r, voff + row * w.rowb, 0, kCpolNT);
}
__device__ __forceinline__ uint4 win_load(const OutWin& w, uint32_t voff, uint32_t row) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(w.r, voff + row * w.rowb, 0, kCpolNT));
}

template <int KIND, int BM>
__device__ __forceinline__ void epilogue(const GemmParams& P, const TileInfo& ti, int wm, int wn, int wave, int lane,
                                         const f32x16_t (&acc)[MT][NTT], char* stage) {
  // The lane index passes through an opaque move so that the epilogue's
  // per-lane address arithmetic stays here instead of being hoisted out of
  // the tile loop, where it would hold registers through every K step.
  asm volatile("" : "+v"(lane));
  // Top-1 row map (KIND_NT, KIND_NN): both rounds' row targets (and, for the
  // combine, the rows' router weights) are loaded before the first store.
  // One counter tracks this wave's loads and stores in issue order, so a load
  // issued after the first round's stores would wait for them as well.
  // Targets outside [0, M) are not written.
  const bool mapped = (KIND == KIND_NT || KIND == KIND_NN) && P.row_tok != nullptr;
  int32_t dst[16];
  float wt[16];
  if constexpr (KIND == KIND_NT || KIND == KIND_NN) {
    if (mapped) {
      // The wave's rows through descriptors that end at the group's last row.
      const int64_t r0 = ti.row0 + wm * WROWS;
      const int32_t nrows = (int32_t)(ti.row_end - r0 < 0 ? 0 : (ti.row_end - r0 > WROWS ? WROWS : ti.row_end - r0));
      const __amdgpu_buffer_rsrc_t rt = make_rsrc(P.row_tok + r0, (uint64_t)nrows * 4);
      const __amdgpu_buffer_rsrc_t rw = make_rsrc(P.row_w + r0, (uint64_t)nrows * 2);
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int r = (q >> 3) * 64 + (q & 7) * 8 + (lane >> 3);
        const int32_t tok = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rt, (uint32_t)r * 4u, 0, 0);
        dst[q] = r < nrows ? tok : -1;
        if constexpr (KIND == KIND_NT) wt[q] = Elt::to_f32(__builtin_amdgcn_raw_buffer_load_b16(rw, (uint32_t)r * 2u, 0, 0));
      }
    }
  }
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int64_t rb = wm * WROWS + half * 64;  // first tile row of the round
    if constexpr (KIND == KIND_FC1) {
      // The wave's 64 columns are 32 gate and the matching 32 up columns:
      // first both as bf16 GEMM outputs (gu), then act = bf16(bf16(silu(gate)) * up).
      const int64_t I = P.I;
      const int64_t j0 = (int64_t)ti.ntile * 128 + wn * 32;
      stage_half<2>(stage, wave, lane, half, [&](int mt, int nt, int i) { return acc4(acc[mt][nt], i); });
      const int cc = lane & 7;
      {
        const OutWin w = out_window(P.gu, ti.row0 + rb, ti.row_end, 2 * I);
        const int64_t j = j0 + (cc & 3) * 8;
        const uint32_t voff = j < I ? (uint32_t)(lane >> 3) * w.rowb + (uint32_t)((cc < 4 ? 0 : I) + j) * 2u : kOOB;
#pragma unroll
        for (int q = 0; q < 8; ++q) win_store(w, voff, q * 8, staged_chunk(stage, wave, q * 8 + (lane >> 3), cc));
      }
      stage_half<1>(stage, wave, lane, half, [&](int mt, int, int i) {
        float g[4], u[4];
#pragma unroll
        for (int k = 0; k < 4; k += 2) {
          g[k] = acc[mt][0][i + k], g[k + 1] = acc[mt][0][i + k + 1];
          u[k] = acc[mt][1][i + k], u[k + 1] = acc[mt][1][i + k + 1];
          Elt::round2(g[k], g[k + 1]);
          Elt::round2(u[k], u[k + 1]);
          g[k] = silu_f32(g[k]), g[k + 1] = silu_f32(g[k + 1]);
          Elt::round2(g[k], g[k + 1]);
        }
        return pack4(g[0] * u[0], g[1] * u[1], g[2] * u[2], g[3] * u[3]);
      });
      const int c4 = lane & 3;
      {
        const OutWin w = out_window(P.act, ti.row0 + rb, ti.row_end, I);
        const int64_t j = j0 + c4 * 8;
        const uint32_t voff = j < I ? (uint32_t)(lane >> 2) * w.rowb + (uint32_t)j * 2u : kOOB;
#pragma unroll
        for (int q = 0; q < 4; ++q) win_store(w, voff, q * 16, staged_chunk(stage, wave, q * 16 + (lane >> 2), c4));
      }
    } else if constexpr (KIND == KIND_NNS) {
      // fc2 dgrad: the tile is dact (bf16, as the reference stores it) for
      // columns j < I; with the forward's gate/up of the same rows it becomes
      // [d_gate | d_up] of dG1.  The round's gate/up loads go out first, so
      // that their latency overlaps the staging.
      // gate/up (gin) and [d_gate | d_up] (c0) share one row layout.
      const int64_t I = P.I;
      const int cc = lane & 7;
      const int64_t j = (int64_t)ti.ntile * BN + wn * WCOLS + cc * 8;
      const OutWin wi = out_window(P.gin, ti.row0 + rb, ti.row_end, 2 * I);
      const OutWin wo = out_window(P.c0, ti.row0 + rb, ti.row_end, 2 * I);
      const uint32_t vg = j < I ? (uint32_t)(lane >> 3) * wi.rowb + (uint32_t)j * 2u : kOOB;
      const uint32_t vu = vg + (uint32_t)I * 2u;
      uint4 gv[8], uv[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        gv[q] = win_load(wi, vg, q * 8);
        uv[q] = win_load(wi, vu, q * 8);
      }
      stage_half<NTT>(stage, wave, lane, half, [&](int mt, int nt, int i) { return acc4(acc[mt][nt], i); });
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint4 v = staged_chunk(stage, wave, q * 8 + (lane >> 3), cc);
        float d[8], g[8], u[8], dg[8], du[8];
        unpack8e<Elt>(v, d);
        unpack8e<Elt>(gv[q], g);
        unpack8e<Elt>(uv[q], u);
        swiglu_bwd8<Elt>(d, g, u, dg, du);
        win_store(wo, vg, q * 8, pack8e<Elt>(dg));
        win_store(wo, vu, q * 8, pack8e<Elt>(du));
      }
    } else if constexpr (KIND == KIND_TN) {
      stage_half<NTT>(stage, wave, lane, half, [&](int mt, int nt, int i) { return acc4(acc[mt][nt], i); });
      const int cc = lane & 7;  // 16-byte chunk (8 columns) of the wave's 64
      const int64_t col = (int64_t)ti.ntile * BN + wn * WCOLS + cc * 8;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int rl = q * 8 + (lane >> 3);
        const uint4 v = staged_chunk(stage, wave, rl, cc);
        const int64_t m = (int64_t)ti.mtile * BM + rb + rl;
        if (m < P.M && col < P.N) {
          bf16_t* crow = m < P.csplit ? P.c0 + ti.g * P.cgs + m * P.ldc : P.c1 + ti.g * P.cgs + (m - P.csplit) * P.ldc;
          st_stream(crow + col, v);
        }
      }
    } else {
      const int cc = lane & 7;  // 16-byte chunk (8 columns) of the wave's 64
      const int64_t col = (int64_t)ti.ntile * BN + wn * WCOLS + cc * 8;
      stage_half<NTT>(stage, wave, lane, half, [&](int mt, int nt, int i) { return acc4(acc[mt][nt], i); });
      const OutWin w = out_window(P.c0, ti.row0 + rb, ti.row_end, P.ldc);
      const uint32_t voff = col < P.N ? (uint32_t)(lane >> 3) * w.rowb + (uint32_t)col * 2u : kOOB;
      // Mapped rows go to row dst of the whole output (dst is -1 for rows
      // past the tile's group): through one descriptor over the output when
      // it spans at most 2 GiB, else through 64-bit addresses.
      const bool whole = (uint64_t)P.M * (uint64_t)P.ldc * 2u <= 0x7fffffffull;
      const OutWin wd = {make_rsrc(KIND == KIND_NT ? P.cout : P.c0, (uint64_t)P.M * P.ldc * 2), w.rowb};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint4 v = staged_chunk(stage, wave, q * 8 + (lane >> 3), cc);
        if (!(KIND == KIND_NN && mapped)) win_store(w, voff, q * 8, v);
        const int32_t d = dst[half * 8 + q];
        if ((KIND == KIND_NT || KIND == KIND_NN) && mapped && whole) {
          const uint32_t vd = col < P.N && (uint32_t)d < (uint32_t)P.M ? (uint32_t)d * wd.rowb + (uint32_t)col * 2u : kOOB;
          if (KIND == KIND_NN) {
            win_store(wd, vd, 0, v);
          } else {
            float f[8];
            unpack8e<Elt>(v, f);
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = __builtin_fmaf(f[j], wt[half * 8 + q], 0.f);
            win_store(wd, vd, 0, pack8e<Elt>(f));
          }
        } else if ((KIND == KIND_NT || KIND == KIND_NN) && mapped && col < P.N && (uint32_t)d < (uint32_t)P.M) {
          if (KIND == KIND_NN) {
            st_stream(P.c0 + (int64_t)d * P.ldc + col, v);
          } else {
            // The weighted combine of a top-1 row, as the combine kernel
            // rounds it: 0 + bf16(f * w).  The fma's single rounding of
            // f * w + 0 is the product's, with -0 made +0, and pack8 rounds
            // it to bf16.
            float f[8];
            unpack8e<Elt>(v, f);
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = __builtin_fmaf(f[j], wt[half * 8 + q], 0.f);
            st_stream(P.cout + (int64_t)d * P.ldc + col, pack8e<Elt>(f));
          }
        }
      }
    }
    // Keep each round's loads and stores in their round (register pressure).
    asm volatile("" ::: "memory");
  }
}

// The partial last K-tile of a K of `K` (-1 if none) and its valid k.
__device__ __forceinline__ void k_tail(int64_t K, int32_t& ktail, int32_t& krem) {
  const int32_t kt_last = (int32_t)((K - 1) / BK);
  krem = (int32_t)(K - (int64_t)kt_last * BK);  // a multiple of 8
  ktail = krem < BK ? kt_last : -1;
}

// Per-lane offsets of a K-contiguous operand whose tile rows start at the
// descriptor base (rows past the descriptor's end fail the range check).
template <int R>
__device__ __forceinline__ void kc_offsets(Operand& op, int wave, int lane, int64_t K) {
  int32_t krem;
  k_tail(K, op.ktail, krem);
  op.tmask = 0;
#pragma unroll
  for (int q0 = 0; q0 < loads_per_wave<R>(); ++q0) {
    const int row = (q0 * NWAVES + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ kc_swz(row);
    op.voff[q0] = (uint32_t)row * op.ldb + (uint32_t)c * 16u;
    op.tmask |= (c * 8 < krem ? 1u : 0u) << q0;
  }
}

// Per-lane offsets of an M/N-contiguous operand, relative to the first k-row
// of each instruction (REBASE: of the K-tile), columns col0.. of the tile.
// Not REBASE: tmask also masks the k-rows past K of the last K-tile.
template <int W, bool REBASE>
__device__ __forceinline__ void mn_offsets(Operand& op, int wave, int lane, int64_t col0, int64_t ncols, int64_t K) {
  constexpr int CH = W / 8, ROWS = 1024 / (2 * W);
  int32_t krem = BK;
  op.ktail = -1;
  if constexpr (!REBASE) k_tail(K, op.ktail, krem);
  op.tmask = 0;
#pragma unroll
  for (int q0 = 0; q0 < loads_per_wave<W>(); ++q0) {
    const int q = q0 * NWAVES + wave;
    const int kk = lane / CH;  // k-row within the instruction
    const int krow = q * ROWS + kk;
    const int c = (lane % CH) ^ (4 * (krow & 3));
    const int64_t col = col0 + c * 8;
    const uint32_t r = REBASE ? krow : kk;
    op.voff[q0] = col < ncols ? r * op.ldb + (uint32_t)col * 2u : kOOB;
    op.tmask |= (krow < krem ? 1u : 0u) << q0;
  }
}

// Describe the operands of one output tile.  FAST weight gradients address
// each operand through one descriptor over the group's rows.
template <int KIND, int BM, bool FAST = false>
__device__ __forceinline__ void setup_operands(const GemmParams& P, Tile<KIND, BM>& tc, int wave, int lane) {
  // Opaque lane: keeps the per-lane offset arithmetic here (see epilogue).
  asm volatile("" : "+v"(lane));
  const TileInfo& ti = tc.i;
  if constexpr (KIND == KIND_TN) {
    // A: the group's rows, columns m of the tile; B: the group's rows, columns n.
    const int64_t rows = ti.row_end - ti.row0;
    tc.A.base = reinterpret_cast<const char*>(P.a.p0 + (int64_t)ti.row0 * P.a.ld);
    tc.A.ldb = (uint32_t)(P.a.ld * 2);
    tc.A.bytes = (uint64_t)rows * (uint64_t)P.a.ld * 2u;
    tc.B.base = reinterpret_cast<const char*>(P.b.p0 + (int64_t)ti.row0 * P.b.ld);
    tc.B.ldb = (uint32_t)(P.b.ld * 2);
    tc.B.bytes = (uint64_t)rows * (uint64_t)P.b.ld * 2u;
    mn_offsets<BM, true>(tc.A, wave, lane, (int64_t)ti.mtile * BM, P.M, 0);
    mn_offsets<BN, true>(tc.B, wave, lane, (int64_t)ti.ntile * BN, P.N, 0);
    if constexpr (FAST) {
      tc.A.r0 = make_rsrc(tc.A.base, tc.A.bytes);
      tc.B.r0 = make_rsrc(tc.B.base, tc.B.bytes);
    } else {
      rebase_ktile(tc.A, 0, true);
      rebase_ktile(tc.B, 0, true);
    }
  } else {
    const int64_t rows = ti.row_end - ti.row0 < BM ? ti.row_end - ti.row0 : BM;
    const bf16_t* a0 = P.a.p0 + (int64_t)ti.row0 * P.a.ld;
    tc.A.base = reinterpret_cast<const char*>(a0);
    tc.A.r0 = tc.A.r1 = make_rsrc(a0, (uint64_t)rows * P.a.ld * 2);
    tc.A.ldb = (uint32_t)(P.a.ld * 2);
    kc_offsets<BM>(tc.A, wave, lane, P.K);
    const bf16_t* b0 = P.b.p0 + (int64_t)ti.g * P.b.gs0;
    const bf16_t* b1 = P.b.p1 + (int64_t)ti.g * P.b.gs1;
    tc.B.base = reinterpret_cast<const char*>(b0);
    if constexpr (KIND == KIND_FC1) {
      // virtual B rows: per 64 rows, 32 gate rows then 32 up rows.  A wave's
      // instructions q = q0*NWAVES + wave fill rows 8q .. 8q+7, which are up
      // rows exactly when bit 2 of the wave index is set, whatever q0: each
      // wave needs only one of the two descriptors, kept in r0.
      tc.B.r0 = make_rsrc(((wave >> 2) & 1) ? b1 : b0, (uint64_t)P.I * P.K * 2);
      tc.B.r1 = tc.B.r0;
      tc.B.ldb = (uint32_t)(P.K * 2);
      int32_t krem;
      k_tail(P.K, tc.B.ktail, krem);
      const int64_t j0 = (int64_t)ti.ntile * 128;
      tc.B.tmask = 0;
#pragma unroll
      for (int q0 = 0; q0 < loads_per_wave<BN>(); ++q0) {
        const int row = (q0 * NWAVES + wave) * 8 + (lane >> 3);
        const int c = (lane & 7) ^ kc_swz(row);
        const int64_t j = j0 + (row >> 6) * 32 + (row & 31);
        tc.B.voff[q0] = j < P.I ? (uint32_t)j * tc.B.ldb + (uint32_t)c * 16u : kOOB;
        tc.B.tmask |= (c * 8 < krem ? 1u : 0u) << q0;
      }
    } else if constexpr (KIND == KIND_NT) {
      // rows n of B[g] ([N][K]) from row ntile*BN on
      const int64_t n0 = (int64_t)ti.ntile * BN;
      tc.B.r0 = tc.B.r1 = make_rsrc(b0 + n0 * P.K, (uint64_t)(P.N - n0) * P.K * 2);
      tc.B.ldb = (uint32_t)(P.K * 2);
      kc_offsets<BN>(tc.B, wave, lane, P.K);
    } else {
      // B[g] is [K][N]; k-rows below split come from b0, the rest from b1
      const int64_t split = P.b.split < P.K ? P.b.split : P.K;
      tc.B.r0 = make_rsrc(b0, (uint64_t)split * P.N * 2);
      tc.B.r1 = make_rsrc(b1, (uint64_t)(P.K - split) * P.N * 2);
      tc.B.split = (int32_t)split;
      tc.B.ldb = (uint32_t)(P.N * 2);
      tc.B.split_bytes = (uint32_t)split * tc.B.ldb;
      mn_offsets<BN, false>(tc.B, wave, lane, (int64_t)ti.ntile * BN, P.N, P.K);
    }
  }
}

// Zero gradient tile of an empty group (wgrad): 16-byte stores, no LDS.
template <int BM, int NT = NTHREADS>
__device__ __forceinline__ void zero_tile(const GemmParams& P, const TileInfo& ti, int t) {
  const uint4 z = make_uint4(0, 0, 0, 0);
  for (int e = t; e < BM * (BN / 8); e += NT) {
    const int64_t m = (int64_t)ti.mtile * BM + e / (BN / 8);
    const int64_t n = (int64_t)ti.ntile * BN + (e % (BN / 8)) * 8;
    if (m < P.M && n < P.N) {
      bf16_t* crow = m < P.csplit ? P.c0 + ti.g * P.cgs + m * P.ldc : P.c1 + ti.g * P.cgs + (m - P.csplit) * P.ldc;
      *reinterpret_cast<uint4*>(crow + n) = z;
    }
  }
}

// Tile order: bands of kBand consecutive m-tiles, walked n-tile by n-tile
// (m fastest).  The 32 blocks of one XCD, which run consecutive tiles, then
// cover 8 m-tiles x 4 n-tiles and share both operands through that XCD's L2:
// 8 A + 4 B strips (128 KB per K-tile) instead of the 1-2 A + 16-28 B strips
// of an n-fastest order over wide outputs.  (PMX_BAND / PMX_BAND_TN: other
// band heights, for measurements.)
#ifndef PMX_BAND
#define PMX_BAND 8
#endif
#ifndef PMX_BAND_TN
#define PMX_BAND_TN PMX_BAND
#endif
#ifndef PMX_BAND_NNS
#define PMX_BAND_NNS PMX_BAND
#endif
template <int KIND>
constexpr int64_t band_height() {
  return KIND == KIND_TN ? PMX_BAND_TN : KIND == KIND_NNS ? PMX_BAND_NNS : PMX_BAND;
}
static_assert(PMX_BAND >= 1 && PMX_BAND <= 32 && PMX_BAND_TN >= 1 && PMX_BAND_TN <= 32 && PMX_BAND_NNS >= 1 &&
                  PMX_BAND_NNS <= 32,
              "band height");

template <int64_t kBand>
__device__ __forceinline__ void band_order(int64_t t, int64_t mtiles, int64_t ntn, int64_t& m, int64_t& n) {
  const int64_t band = t / (kBand * ntn);
  const int64_t m0 = band * kBand;
  const int64_t gm = mtiles - m0 < kBand ? mtiles - m0 : kBand;
  const int64_t r = t - m0 * ntn;
  n = r / gm;
  m = m0 + (r - n * gm);
}

// The tile list: every kind but TN walks m-tiles of all groups (exclusive
// prefix `tpre`, ntn n-tiles each); TN walks the tiles_per_group weight tiles
// of each group, whose K is the group's row count.  `local` >= 0 (TN only)
// names tile `local` of group `tile` instead of a position in the list.
// UNI: `tile` is uniform over the wave and the result is made so; else each
// lane decodes its own tile (the block's tile table, filled at kernel start).
template <int KIND, int BM, bool UNI = true>
__device__ __forceinline__ TileInfo decode_tile(const GemmParams& P, int64_t tile, const int32_t* tpre, int G,
                                                int64_t ntn, int64_t tiles_per_group, int64_t local = -1) {
  auto rd = [](int32_t v) { return UNI ? uni(v) : v; };
  TileInfo ti;
  int64_t m, n;
  if constexpr (KIND == KIND_TN) {
    int64_t g = tile;
    if (local < 0) {
      g = tile / tiles_per_group;
      local = tile - g * tiles_per_group;
    }
    band_order<band_height<KIND>()>(local, tiles_per_group / ntn, ntn, m, n);
    ti.g = (int32_t)g;
    ti.mtile = (int32_t)m;
    ti.row0 = P.offsets[g];
    ti.row_end = P.offsets[g + 1];
    ti.nk = (int32_t)(((int64_t)ti.row_end - ti.row0 + BK - 1) / BK);
  } else {
    band_order<band_height<KIND>()>(tile, tpre[G], ntn, m, n);
    // Uniform binary search for the group holding m-tile m.
    int lo = 0, hi = G;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (rd(tpre[mid]) <= m) lo = mid;
      else hi = mid - 1;
    }
    ti.g = lo;
    ti.mtile = (int32_t)m - rd(tpre[lo]);
    ti.row0 = P.offsets[lo] + ti.mtile * BM;
    ti.row_end = P.offsets[lo + 1];
    ti.nk = (int32_t)((P.K + BK - 1) / BK);
  }
  ti.ntile = (int32_t)n;
  ti.g = rd(ti.g);
  ti.mtile = rd(ti.mtile);
  ti.ntile = rd(ti.ntile);
  ti.row0 = rd(ti.row0);
  ti.row_end = rd(ti.row_end);
  ti.nk = rd(ti.nk);
  return ti;
}

// Wait until at most PENDING of this wave's vector memory operations (its
// buffer->LDS loads, and any stores since) are in flight.
template <int PENDING>
__device__ __forceinline__ void wait_loads() {
  static_assert(PENDING >= 0 && PENDING <= 63, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PENDING) : "memory");
}

// Same, and this wave's LDS reads and writes have completed.
template <int PENDING>
__device__ __forceinline__ void wait_loads_lds() {
  static_assert(PENDING >= 0 && PENDING <= 63, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(PENDING) : "memory");
}

// Wait until this wave's LDS reads and writes have completed.
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Workgroup barrier that neither the compiler's memory model nor its
// scheduler moves anything across: memory operations stay on their side (the
// asm clobbers memory), and so do the MFMAs, so that every LDS read consumed
// before the barrier has returned by the time the wave reaches it.
__device__ __forceinline__ void block_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Weight-gradient schedule.  A wgrad tile of copy g costs ceil(rows_g / 64)
// K-tiles, so copies of very different sizes make the round-robin deal of
// tiles to blocks uneven.  The schedule keeps the deal's structure - the
// tile list cut into bands of 32 tiles, the 8 m x 4 n tiles that one XCD's
// 32 blocks multiply side by side sharing operand strips in its L2, and all
// XCDs working on the 8 neighbouring bands of one round at the same time,
// which lets the XCDs share the K-tile rows in flight through the
// memory-side cache - and changes two things:
//   - copies are ordered by K-tile count, largest first, so that the bands
//     of a round cost about the same and fall in cost within the round;
//   - within each round the XCD with the most K-tiles dealt so far takes the
//     cheapest band, the next one the next cheapest, and so on (the deal is
//     worked out once per block, before its first tile).
// (A longest-processing-time deal of bands to XCDs across rounds balances
// the work as well but lets the XCDs drift apart over different copies'
// rows; measured slower on every shape.  Alternating the direction of the
// deal from round to round keeps the rounds but balances less: on the
// DeepSeek-V3-shape share 96% against 98% of the mean per block.)  Needs a
// grid of whole XCDs and G <= NT (the block's threads); otherwise (false) the plain order
// is used.  Rounds past what the LDS holds alternate direction.
constexpr int kBandTiles = 32;
constexpr int kNumXcd = 8;

// `order[r]` = the copy of rank r (more K-tiles first, ties by copy index);
// `deal[r]` (bytes after nk[G]) = the band of round r, 0..7 within the round,
// that XCD `xcd` takes, for the first `cap` rounds (the return value).
// `costs` is scratch of `cost_slots` int32 (LDS not yet in use).
template <int NT = NTHREADS>
__device__ __noinline__ int32_t build_wgrad_order(const GemmParams& P, int32_t* nk, int32_t* order, int t,
                                                  int64_t total, int64_t tiles_per_group, int32_t xcd,
                                                  int32_t* costs, int32_t cost_slots) {
  const int G = P.G;
  if (t < G) nk[t] = (int32_t)(((int64_t)P.offsets[t + 1] - P.offsets[t] + BK - 1) / BK);
  __syncthreads();
  if (t < G) {
    const int32_t mine = nk[t];
    int32_t rank = 0;
    for (int g = 0; g < G; ++g) {
      const int32_t v = nk[g];
      rank += (v > mine || (v == mine && g < t)) ? 1 : 0;
    }
    order[rank] = t;
  }
  __syncthreads();
  // Cost of every band: the K-tiles of its first tile's copy (the dearest of
  // the band: copies come largest first); 0 past the last tile.
  const int64_t bands = (total + kBandTiles - 1) / kBandTiles;
  const int64_t rounds = (bands + kNumXcd - 1) / kNumXcd;
  int64_t cap = (int64_t)(kMaxGroups + 1 - G) * 4;
  if (cap > cost_slots / kNumXcd) cap = cost_slots / kNumXcd;
  if (cap > rounds) cap = rounds;
  for (int64_t b = t; b < cap * kNumXcd; b += NT) {
    const int64_t tile = b * kBandTiles;
    costs[b] = tile < total ? nk[order[tile / tiles_per_group]] : 0;
  }
  __syncthreads();
  if (t < 64) {
    // Lanes 0..7 stand for the XCDs; `cum` = K-tiles dealt to XCD `t`.
    unsigned char* deal = reinterpret_cast<unsigned char*>(nk + G);
    int32_t cum = 0;
    for (int32_t r = 0; r < (int32_t)cap; ++r) {
      const int32_t cost = t < kNumXcd ? costs[r * kNumXcd + t] : 0;
      int32_t rank = 0;  // XCDs with more K-tiles so far (ties: lower index)
#pragma unroll
      for (int y = 0; y < kNumXcd; ++y) {
        const int32_t cy = __builtin_amdgcn_readlane(cum, y);
        rank += (cy > cum || (cy == cum && y < t)) ? 1 : 0;
      }
      const int32_t band = rank < kNumXcd ? kNumXcd - 1 - rank : 0;
      cum += __shfl(cost, band);
      if (t == xcd) deal[r] = (unsigned char)band;
    }
  }
  __syncthreads();
  return (int32_t)cap;
}

// Exclusive prefix of m-tiles (BM rows) per group into tpre[0..G]: GPT groups
// per thread, then a block scan of the NT partial sums in scan_buf.
template <int BM, int NT>
__device__ __forceinline__ void group_prefix(const GemmParams& P, int32_t* tpre, int32_t* scan_buf, int t) {
  constexpr int GPT = kMaxGroups / NT;
  const int G = P.G;
  int32_t loc[GPT];
  int32_t sum = 0;
#pragma unroll
  for (int i = 0; i < GPT; ++i) {
    const int g = t * GPT + i;
    int32_t v = 0;
    if (g < G) v = (P.offsets[g + 1] - P.offsets[g] + BM - 1) / BM;
    loc[i] = sum;
    sum += v;
  }
  scan_buf[t] = sum;
  __syncthreads();
  for (int off = 1; off < NT; off <<= 1) {
    const int32_t add = t >= off ? scan_buf[t - off] : 0;
    __syncthreads();
    scan_buf[t] += add;
    __syncthreads();
  }
  const int32_t base = scan_buf[t] - sum;
#pragma unroll
  for (int i = 0; i < GPT; ++i) {
    const int g = t * GPT + i;
    if (g < G) tpre[g] = base + loc[i];
  }
  if (t == NT - 1) tpre[G] = scan_buf[NT - 1];
  __syncthreads();
}

// One block per CU walks its tiles (slot, slot + grid, ...) as one stream of
// 64-deep K-tiles through two LDS stages: K-tile p of the stream is
// multiplied from one stage while K-tile p+1 lands in the other.
//
// Between barrier p-1 (after which stream K-tile p is in LDS and every wave
// has finished reading K-tile p-1) and barrier p, a wave
//   - issues its loads of K-tile p+1 into the stage of K-tile p-1, one per
//     MFMA pair of the first two k-steps (per MFMA of the first k-step for
//     the wgrad), so that they have the rest of the K-tile to land,
//   - multiplies the four 16-deep k-steps, reading each k-step's fragments
//     during the previous k-step's MFMAs (k-step 0's during k-step 3 of
//     K-tile p-1), so that LDS latency hides behind MFMAs,
//   - waits for its loads and its LDS reads, then passes barrier p.
// At the end of an output tile the next stream K-tile is issued into the
// stage just freed before the tile's last k-step is multiplied and the tile
// is written out (through per-wave epilogue regions outside the stages), so
// the loads stay in flight across the epilogue.
// BAL (weight gradient only): the balanced band order of build_wgrad_order;
// the host picks it when the grid is 8 XCDs x 32 blocks and G <= NTHREADS.
// FAST (ragged-M kinds): K is a multiple of 64 and the dgrad weights are one
// tensor, so the loads need no K-tail masking, no split test and no `live`
// test (dma_kc, dma_mn; the slots past the block's last K-tile re-load the
// first K-tile of its last tile, whose data is never multiplied).  FAST
// weight gradient: every operand row lies within 31-bit offsets, so each
// group is one descriptor and a K-tile is a scalar offset into it, instead of
// a 64-bit window rebased per K-tile.
// RS (FAST fc1, fc2 and fc1 dgrad): no buffer->LDS loads.  Each of the
// wave's eight 1 KB pieces of a K-tile passes through one register: at its
// own point of K-tile p (one every four MFMA groups) the piece of K-tile p+1
// is written to the refill stage and the register re-loaded with K-tile
// p+2, so every load has a whole K-tile to land and the loads are spread
// over the K-tile instead of crowding its first half; the compiler tracks
// these loads, and the end of a K-tile waits only for LDS.
template <int KIND, int BM, bool BAL = false, bool FAST = false, bool RS = false>
__global__ __launch_bounds__(NTHREADS, 1) void grouped_gemm_kernel(GemmParams P) {
  static_assert(!BAL || KIND == KIND_TN, "the balanced order is the weight gradient's");
  static_assert(!RS || (FAST && (KIND == KIND_FC1 || KIND == KIND_NT || KIND == KIND_NN)),
                "register-staged operands: FAST ragged-M kinds without the SwiGLU backward");
  static_assert(BM == 256, "the schedule below is written for 256 x 256 tiles");
  static_assert(BK == pmx::kKTileRows, "wgrad K-tile windows are 64 rows deep");
  constexpr int STAGE_BYTES = (BM + BN) * BK * 2;
  constexpr int QA = loads_per_wave<BM>(), QB = loads_per_wave<BN>();  // per wave and K-tile
  __shared__ __attribute__((aligned(1024))) char lds[NSTAGE * STAGE_BYTES];
  __shared__ int32_t tpre[kMaxGroups + 1];
  __shared__ int32_t scan_buf[NTHREADS];
  __shared__ int4 ttab[kTileTab];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = uni(t >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int G = P.G;

  const int64_t grid = gridDim.x;
  const int32_t xcd = (int32_t)(blockIdx.x % kNumXcd);
  const int32_t xj = (int32_t)(blockIdx.x / kNumXcd);  // the block's position in its XCD's bands
  int64_t ntn, tiles_per_group = 0, total;
  int32_t deal_rounds = 0;  // BAL: rounds whose band comes from the deal table
  if constexpr (KIND == KIND_TN) {
    const int64_t mtn = (P.M + BM - 1) / BM;
    ntn = (P.N + BN - 1) / BN;
    tiles_per_group = mtn * ntn;
    total = tiles_per_group * G;
    if constexpr (BAL) {
      deal_rounds = uni(build_wgrad_order(P, tpre, scan_buf, t, total, tiles_per_group, xcd,
                                          reinterpret_cast<int32_t*>(lds), (int32_t)(sizeof(lds) / sizeof(int32_t))));
    }
  } else {
    ntn = (KIND == KIND_FC1) ? (P.I + 127) / 128 : (P.N + BN - 1) / BN;
    group_prefix<BM, NTHREADS>(P, tpre, scan_buf, t);
    total = (int64_t)tpre[G] * ntn;
  }

  // XCD-aware order: blocks are dispatched round-robin over the 8 XCDs, so
  // give the blocks of one XCD a contiguous run of each wave of tiles.
  int64_t slot = blockIdx.x;
  if ((grid & 7) == 0) slot = (blockIdx.x & 7) * (grid >> 3) + (blockIdx.x >> 3);

  // The block's seq-th output tile; false past its last.  Plain order: tiles
  // slot, slot + grid, ...  Balanced wgrad order (BAL, grid = 8 XCDs x 32
  // blocks): copies by rank; in round seq, this block's XCD takes band
  // 8 seq + deal[seq] (past the table: 8 seq + x, or 8 seq + 7 - x when seq
  // is odd) and its block j tile j of it.
  const unsigned char* deal = reinterpret_cast<const unsigned char*>(tpre + G);

  // The block's first kTileTab tiles, decoded at once by its threads into LDS
  // (entry s: the block's s-th tile; mtile -1 past its last), so that moving
  // on to the next tile costs one LDS read instead of a chain of dependent
  // divisions, LDS reads and offset loads.  A block has at most
  // ceil(total / grid) tiles in either order.
  const int64_t rounds = (total + grid - 1) / grid;
  const int32_t ntab = (int32_t)(rounds < kTileTab ? rounds : kTileTab);
  const int32_t nk_all = KIND == KIND_TN ? 0 : (int32_t)((P.K + BK - 1) / BK);
  for (int e = t; e < ntab; e += NTHREADS) {
    TileInfo d;
    bool ok;
    if constexpr (!BAL) {
      const int64_t tile = slot + (int64_t)e * grid;
      ok = tile < total;
      if (ok) d = decode_tile<KIND, BM, false>(P, tile, tpre, G, ntn, tiles_per_group);
    } else {
      const int32_t x = e < deal_rounds ? (int32_t)deal[e] : ((e & 1) ? kNumXcd - 1 - xcd : xcd);
      const int64_t tile = ((int64_t)e * kNumXcd + x) * kBandTiles + xj;
      ok = tile < total;
      if (ok) {
        const int64_t rank = tile / tiles_per_group;
        d = decode_tile<KIND, BM, false>(P, scan_buf[rank], tpre, G, ntn, tiles_per_group,
                                         tile - rank * tiles_per_group);
      }
    }
    ttab[e] = ok ? make_int4(d.row0, d.row_end, d.g | (d.ntile << 12), d.mtile) : make_int4(0, 0, 0, -1);
  }
  __syncthreads();

  auto tile_at = [&](int64_t seq, TileInfo& ti) -> bool {
    if (seq < ntab) {
      const int4 e = ttab[seq];
      if (uni(e.w) < 0) return false;
      ti.row0 = uni(e.x);
      ti.row_end = uni(e.y);
      ti.g = uni(e.z) & 0xfff;
      ti.ntile = uni(e.z) >> 12;
      ti.mtile = uni(e.w);
      ti.nk = KIND == KIND_TN ? (int32_t)(((int64_t)ti.row_end - ti.row0 + BK - 1) / BK) : nk_all;
      return true;
    }
    if constexpr (!BAL) {
      const int64_t tile = slot + seq * grid;
      if (tile >= total) return false;
      ti = decode_tile<KIND, BM>(P, tile, tpre, G, ntn, tiles_per_group);
      return true;
    } else {
      const int32_t x = seq < deal_rounds ? uni((int32_t)deal[seq]) : ((seq & 1) ? kNumXcd - 1 - xcd : xcd);
      const int64_t tile = (seq * kNumXcd + x) * kBandTiles + xj;
      if (tile >= total) return false;
      const int64_t rank = tile / tiles_per_group;
      ti = decode_tile<KIND, BM>(P, uni(scan_buf[rank]), tpre, G, ntn, tiles_per_group,
                                 tile - rank * tiles_per_group);
      return true;
    }
  };

  // Consume cursor: the output tile being multiplied.  Tiles without K-tiles
  // (wgrad of an empty group) are written as zeros on the way.
  int64_t c_seq = 0;
  TileInfo cur;
  for (;; ++c_seq) {
    if (!tile_at(c_seq, cur)) return;
    if (cur.nk > 0) break;
    zero_tile<BM>(P, cur, t);
  }

  // Issue cursor: one K-tile in front, over the same tile sequence.  Past the
  // block's last K-tile it issues through an empty descriptor (zeros).
  Tile<KIND, BM> it;
  int64_t i_seq = c_seq;
  int32_t i_kt = 0;
  bool i_live = true;
  it.i = cur;
  setup_operands<KIND, BM, FAST>(P, it, wave, lane);
  auto advance_issue = [&]() {
    if (!i_live) return;
    if (++i_kt < it.i.nk) {
      if constexpr (KIND == KIND_TN && !FAST) {
        rebase_ktile(it.A, i_kt, true);
        rebase_ktile(it.B, i_kt, true);
      }
      return;
    }
    i_kt = 0;
    while (tile_at(++i_seq, it.i)) {
      if (it.i.nk > 0) {
        setup_operands<KIND, BM, FAST>(P, it, wave, lane);
        return;
      }
    }
    i_live = false;
    if constexpr (KIND == KIND_TN && !FAST) {
      rebase_ktile(it.A, 0, false);
      rebase_ktile(it.B, 0, false);
    }
  };
  auto issue_next = [&](char* stage) {
    issue_stage<KIND, BM, FAST>(stage, it, i_kt, i_live, wave);
    advance_issue();
  };

  // RS: one register per piece of this wave's share of a K-tile.  During
  // K-tile p each piece is written to the refill stage (K-tile p + 1, loaded
  // a K-tile earlier) and at once re-loaded with K-tile p + 2, at evenly
  // spaced points of the K-tile, so every load has a whole K-tile to land.
  constexpr int NPC = RS ? QA + QB : 1;
  uint4 rg[NPC];
  int cs = 0;  // stage of the K-tile being multiplied
  if constexpr (RS) {
    static_for<0, NPC>([&](auto q) __attribute__((always_inline)) {
      rg[decltype(q)::value] = load_piece<KIND, BM, decltype(q)::value>(it, i_kt, wave);
    });
    advance_issue();
    static_for<0, NPC>([&](auto q) __attribute__((always_inline)) {
      store_piece<BM, decltype(q)::value>(lds, wave, lane, rg[decltype(q)::value]);
      rg[decltype(q)::value] = load_piece<KIND, BM, decltype(q)::value>(it, i_kt, wave);
    });
    advance_issue();
    wait_lds();
    block_barrier();
  } else {
    // Prologue: the first K-tile lands in stage 0, then the second is issued.
    issue_next(lds);
    wait_loads<0>();
    block_barrier();
    issue_next(lds + STAGE_BYTES);
  }

  // Per k-step: NM MFMAs, one per pinned group, and NR fragment reads, two
  // per group in the first groups.  The next K-tile's QA + QB loads go one
  // every SPREAD-th group from the start of k-step 0: every other group of
  // the first two k-steps, except for the wgrad, whose M/N-contiguous loads
  // go one per group of k-step 0 (measured: +3% on the wgrad, 3-6% slower
  // for the other kinds; spreading over three or four k-steps is slower).
  constexpr int NM = MT * NTT, NR = MT + NTT, PER = 1, NF = NM;
  constexpr int SPREAD = KIND == KIND_TN ? 1 : 2;
  static_assert(NR % 2 == 0 && NR / 2 <= NF && QA + QB == NF, "schedule shape");
  f32x16_t acc[MT][NTT];
  Frags<BM> f0, f1;

  // The fragment reads of k-step KS into f: two per MFMA group in the first
  // half of the groups, in the order the MFMAs consume them.
  auto reads_half = [&](auto jj, const char* stage, auto ks, Frags<BM>& f) __attribute__((always_inline)) {
    constexpr int j = decltype(jj)::value;
    if constexpr (2 * j < NR) {
      read_frag<KIND, BM, frag_order(2 * j)>(stage, decltype(ks)::value, wm, wn, lane, f);
      read_frag<KIND, BM, frag_order(2 * j + 1)>(stage, decltype(ks)::value, wm, wn, lane, f);
    }
  };
  // RS: piece i is written and re-loaded at group RSP * i of the K-tile.
  constexpr int RSP = RS ? 4 * NF / NPC : 1;
  auto rs_piece = [&](auto pc, char* refill) __attribute__((always_inline)) {
    constexpr int q = decltype(pc)::value;
    store_piece<BM, q>(refill, wave, lane, rg[q]);
    rg[q] = load_piece<KIND, BM, q>(it, i_kt, wave);
  };
  // k-step KS of the current K-tile: MFMAs of k-step KS-1 (fragments `fm`)
  // interleaved with the reads of k-step KS into `fr`, and, with LOADS, the
  // loads of the next K-tile that fall into this k-step's groups (RS: the
  // pieces that fall into them).  FIRST: k-step KS-1 is the tile's first.
  auto kstep = [&](auto ks, auto loads, auto first, const char* stage, char* refill, const Frags<BM>& fm,
                   Frags<BM>& fr) __attribute__((always_inline)) {
    static_for<0, NF>([&](auto jj) __attribute__((always_inline)) {
      constexpr int j = decltype(jj)::value;
      if constexpr (RS) {
        constexpr int slot = decltype(ks)::value * NF + j;
        if constexpr (slot % RSP == 0 && slot / RSP < NPC) rs_piece(Int<slot / RSP>{}, refill);
      } else if constexpr (decltype(loads)::value) {
        static_for<0, QA + QB>([&](auto ll) __attribute__((always_inline)) {
          constexpr int l = decltype(ll)::value;
          if constexpr (SPREAD * l == decltype(ks)::value * NF + j) {
            if constexpr (l < QA) issue_one<KIND, BM, FAST, 0, l>(refill, it, i_kt, i_live, wave);
            else issue_one<KIND, BM, FAST, 1, l - QA>(refill, it, i_kt, i_live, wave);
          }
        });
      }
      reads_half(jj, stage, ks, fr);
      mma_some<BM, j * PER, PER, decltype(first)::value>(fm, acc);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  for (;;) {
    // Output tile `cur`: its first K-tile is in stage cs, and the next stream
    // K-tile is in flight into the other stage.
    {
      // K-tile 0: no MFMAs pending, and the next K-tile is already in flight.
      const char* stage = lds + cs * STAGE_BYTES;
      char* refill = lds + (cs ^ 1) * STAGE_BYTES;
      if constexpr (RS) {
        // the pieces of k-step 0's groups (that k-step's MFMAs belong to the previous tile)
        static_for<0, NPC>([&](auto pc) __attribute__((always_inline)) {
          if constexpr (decltype(pc)::value * RSP < NF) rs_piece(pc, refill);
        });
      }
      static_for<0, NR>([&](auto jj) __attribute__((always_inline)) {
        constexpr int j = decltype(jj)::value;
        read_frag<KIND, BM, frag_order(j)>(stage, 0, wm, wn, lane, f0);
      });
      kstep(Int<1>{}, Int<0>{}, Int<1>{}, stage, refill, f0, f1);
      kstep(Int<2>{}, Int<0>{}, Int<0>{}, stage, refill, f1, f0);
      kstep(Int<3>{}, Int<0>{}, Int<0>{}, stage, refill, f0, f1);
      if constexpr (RS) {
        advance_issue();
        wait_lds();
      } else {
        wait_loads_lds<0>();
      }
      block_barrier();
      cs ^= 1;
    }
    for (int32_t kt = 1; kt < cur.nk; ++kt) {
      const char* stage = lds + cs * STAGE_BYTES;
      char* refill = lds + (cs ^ 1) * STAGE_BYTES;
      kstep(Int<0>{}, Int<1>{}, Int<0>{}, stage, refill, f1, f0);
      kstep(Int<1>{}, Int<1>{}, Int<0>{}, stage, refill, f0, f1);
      kstep(Int<2>{}, Int<1>{}, Int<0>{}, stage, refill, f1, f0);
      kstep(Int<3>{}, Int<1>{}, Int<0>{}, stage, refill, f0, f1);
      advance_issue();
      if constexpr (RS) {
        wait_lds();
      } else {
        wait_loads_lds<0>();
      }
      block_barrier();
      cs ^= 1;
    }
    // Move the consume cursor on.
    const TileInfo done = cur;
    bool more = false;
    while (tile_at(++c_seq, cur)) {
      if (cur.nk > 0) {
        more = true;
        break;
      }
      zero_tile<BM>(P, cur, t);
    }
    // The stage of the tile's last K-tile is free (barrier above): each wave
    // stages its output in its own chunks of it, then, once its LDS reads
    // have returned, issues the next stream K-tile into the same chunks.
    mma_frags<BM>(f1, acc);
    epilogue<KIND, BM>(P, done, wm, wn, wave, lane, acc, lds + (cs ^ 1) * STAGE_BYTES);
    if (!more) {
      wait_loads<0>();
      return;
    }
    if constexpr (!RS) {
      wait_lds();
      issue_next(lds + (cs ^ 1) * STAGE_BYTES);
    }
  }
}

// ---------------------------------------------------------------------------
// Four-wave kernel (FAST loads only).
//
// The same persistent walk as grouped_gemm_kernel - band order, LDS tile
// table, balanced weight-gradient deal, one stream of 64-deep K-tiles through
// two 64 KB stages filled by buffer->LDS loads - with 4 waves, one per SIMD,
// in a 2 x 2 arrangement, each owning 128 x 128 of the 256 x 256 output tile
// as 8 x 8 tiles of v_mfma_f32_16x16x32_bf16 (256 accumulator registers per
// lane, in AGPRs).  Per K-tile the waves read 128 KB of fragments from LDS
// (the 8-wave layout: 192 KB), and a 16 x 16 accumulator moves half the
// register bytes per flop of a 32 x 32 one, which at the part's power limit
// lets the matrix cores run at a higher clock.  A K-tile is two 32-deep
// k-steps of 64 MFMAs; the MFMAs run one k-step behind the fragment reads, so
// each K-tile's single block barrier falls between two k-steps of MFMAs and
// every wave multiplies from registers right after it.  The next K-tile's 16
// loads per wave go one per MFMA group, half in each k-step.
// ---------------------------------------------------------------------------
namespace w4 {

// Kinds (bit KIND) whose next K-tile's loads all go among the first k-step's
// MFMAs (a whole K-tile less half a k-step to land) instead of half in each
// k-step.  Measured in the layer (config 3 / the Qwen3 shape, ms): fc1 +
// SwiGLU 3.10 -> 3.02-3.05 / 0.85 -> 0.81, fc2 dgrad 1.80 -> 1.74-1.76 /
// 0.53 -> 0.49-0.50, fc1 wgrad 3.31-3.34 -> 2.89-2.90 / 0.82 -> 0.78-0.79.
// Two loads per MFMA group in the first half of the k-step instead: 2-10%
// slower.  (The fc2 forward spills four VGPRs that way; it runs on the
// eight-wave kernel.)
#ifndef PMX_W4_LOADS_FIRST_HALF
#define PMX_W4_LOADS_FIRST_HALF 29
#endif

constexpr int NW = 4, NT = 64 * NW;
constexpr int BM = 256;
constexpr int FM = 8, FN = 8;                // 16 x 16 accumulator tiles per wave
constexpr int QO = BM * BK * 2 / 1024 / NW;  // loads per wave, operand and K-tile (8)
constexpr int STAGE_BYTES = (BM + BN) * BK * 2;
constexpr int B_OFF = BM * BK * 2;  // B's region within a stage
static_assert(BM == BN, "square block tiles");

// M/N-contiguous tiles ([64 k][256]): 16-byte chunk c of k-row kk is stored at
// c ^ mn_swz(kk), so that the 4 k-rows and the two 8-row k-blocks that one
// half-wave's transposing fragment read touches fall on distinct banks.
__device__ __forceinline__ int mn_swz(int kk) { return (4 * (kk & 3)) ^ (2 * ((kk >> 3) & 1)); }

// Operand of one output tile: descriptors and this wave's per-lane load
// offsets.  Load q0 (0 .. QO-1) of a K-tile covers 1 KB of the stage at chunk
// q0 * NW + wave of the operand's region; its per-lane offset is off[q0 & 1]
// and the rest, (q0 >> SHIFT) * step plus the K-tile advance, goes into the
// instruction's scalar offset (SHIFT is 1 for fc1's weights, else 0): no
// per-load vector arithmetic, two offsets per operand.  The range check covers
// the sum of both offsets.  A lane whose chunk lies outside the operand's
// columns holds kOOB; for the weight gradient kOOB plus a large scalar offset
// may wrap into the descriptor, which loads other columns of the operand
// into that lane's slot - they feed only output columns that are never
// written.
struct Op {
  __amdgpu_buffer_rsrc_t r0, r1;  // r1: fc1's up rows (loads with odd q0)
  uint32_t ldb;                   // bytes between consecutive (k-)rows
  uint32_t step;                  // offset per step of q0 >> SHIFT
  uint32_t off[2];                // per-lane offset of loads with even / odd q0
};

template <int KIND>
struct Tile {
  TileInfo i;
  Op A, B;
};

// K-contiguous operand: load q fills rows 8q .. 8q+7, lane i row 8q + i/8,
// physical chunk i%8 = logical chunk ^ kc_swz(row).  With q = q0 * NW + wave
// the row's swizzle does not depend on q0 (kc_swz(row) = (i/16 + 4 wave) % 8),
// so load q0's offset is load 0's plus q0 * 32 rows.
__device__ __forceinline__ void kc_offs(Op& op, int wave, int lane) {
  const int row = wave * 8 + (lane >> 3);
  const int c = (lane & 7) ^ kc_swz(row);
  op.off[0] = op.off[1] = (uint32_t)row * op.ldb + (uint32_t)c * 16u;
  op.step = 32u * op.ldb;
}

// M/N-contiguous operand, columns col0 .. col0+255: load q fills k-rows 2q,
// 2q+1; lane i k-row 2q + i/32, physical chunk i%32 = logical chunk ^
// mn_swz(k-row).  With q = q0 * NW + wave the swizzle depends on q0 only
// through its parity (bit 3 of the k-row), so there are two column offsets.
// KT_ROW: the offset counts the k-row within the K-tile (q0 adds 8 rows);
// else within the load (the K-tile advance includes the load's rows).
template <bool KT_ROW>
__device__ __forceinline__ void mn_offs(Op& op, int wave, int lane, int64_t col0, int64_t ncols) {
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int krow = (par * NW + wave) * 2 + (lane >> 5);
    const int c = (lane & 31) ^ mn_swz(krow);
    const int64_t col = col0 + c * 8;
    const uint32_t r = KT_ROW ? (uint32_t)((wave * 2) + (lane >> 5)) : (uint32_t)(lane >> 5);
    // load q0 = par: its k-row (KT_ROW) is r + 8 * par, counted by the step
    op.off[par] = col < ncols ? r * op.ldb + (uint32_t)col * 2u : kOOB;
  }
  op.step = KT_ROW ? 8u * op.ldb : 0u;
}

// Describe the operands of one output tile (FAST: K a multiple of 64 and the
// dgrad weights one tensor; weight gradient: its operands within 31-bit
// offsets, one descriptor per group).
template <int KIND>
__device__ __forceinline__ void setup(const GemmParams& P, Tile<KIND>& tc, int wave, int lane) {
  asm volatile("" : "+v"(lane));  // keep the per-lane arithmetic here (see epilogue)
  const TileInfo& ti = tc.i;
  if constexpr (KIND == KIND_TN) {
    const int64_t rows = ti.row_end - ti.row0;
    tc.A.ldb = (uint32_t)(P.a.ld * 2);
    tc.B.ldb = (uint32_t)(P.b.ld * 2);
    tc.A.r0 = tc.A.r1 = make_rsrc(P.a.p0 + (int64_t)ti.row0 * P.a.ld, (uint64_t)rows * P.a.ld * 2);
    tc.B.r0 = tc.B.r1 = make_rsrc(P.b.p0 + (int64_t)ti.row0 * P.b.ld, (uint64_t)rows * P.b.ld * 2);
    mn_offs<true>(tc.A, wave, lane, (int64_t)ti.mtile * BM, P.M);
    mn_offs<true>(tc.B, wave, lane, (int64_t)ti.ntile * BN, P.N);
  } else {
    const int64_t rows = ti.row_end - ti.row0 < BM ? ti.row_end - ti.row0 : BM;
    tc.A.ldb = (uint32_t)(P.a.ld * 2);
    tc.A.r0 = tc.A.r1 = make_rsrc(P.a.p0 + (int64_t)ti.row0 * P.a.ld, (uint64_t)rows * P.a.ld * 2);
    kc_offs(tc.A, wave, lane);
    const bf16_t* b0 = P.b.p0 + (int64_t)ti.g * P.b.gs0;
    if constexpr (KIND == KIND_FC1) {
      // Virtual B rows: per 64 rows, 32 gate rows then the matching 32 up rows.
      // Load q covers rows 8q .. 8q+7: block q/8 = q0/2, up rows exactly when
      // q % 8 >= 4, i.e. when q0 is odd; row & 31 = 8 wave + i/8 for every q0.
      // So load q0 reads intermediate row j0 + 32 (q0/2) of the gate (even
      // q0) or up (odd q0) weights, j0 = 128 ntile + 8 wave + i/8; rows past
      // I fail the descriptor's range check.
      tc.B.r0 = make_rsrc(b0, (uint64_t)P.I * P.K * 2);
      tc.B.r1 = make_rsrc(P.b.p1 + (int64_t)ti.g * P.b.gs1, (uint64_t)P.I * P.K * 2);
      tc.B.ldb = (uint32_t)(P.K * 2);
      const int64_t j0 = (int64_t)ti.ntile * 128 + wave * 8 + (lane >> 3);
      const int row = wave * 8 + (lane >> 3);
      const int c = (lane & 7) ^ kc_swz(row);
      tc.B.step = 32u * tc.B.ldb;
      tc.B.off[0] = tc.B.off[1] = j0 < P.I ? (uint32_t)j0 * tc.B.ldb + (uint32_t)c * 16u : kOOB;
    } else if constexpr (KIND == KIND_NT) {
      const int64_t n0 = (int64_t)ti.ntile * BN;
      tc.B.r0 = tc.B.r1 = make_rsrc(b0 + n0 * P.K, (uint64_t)(P.N - n0) * P.K * 2);
      tc.B.ldb = (uint32_t)(P.K * 2);
      kc_offs(tc.B, wave, lane);
    } else {
      // NN / NNS: B[g] is [K][N] in one tensor.
      tc.B.r0 = tc.B.r1 = make_rsrc(b0, (uint64_t)P.K * P.N * 2);
      tc.B.ldb = (uint32_t)(P.N * 2);
      mn_offs<false>(tc.B, wave, lane, (int64_t)ti.ntile * BN, P.N);
    }
  }
}

// Load J of this wave's share of K-tile kt (A: 0 .. QO-1, B: QO .. 2QO-1).
// Every offset stays within its descriptor or fails the range check; kt is
// always a K-tile of the tile (a finished cursor re-loads K-tile 0).
template <int KIND, int J>
__device__ __forceinline__ void issue(char* stage, const Tile<KIND>& tc, int32_t kt, int wave) {
  constexpr int q0 = J % QO;
  const int q = q0 * NW + wave;
  if constexpr (J < QO) {
    const uint32_t soff = KIND == KIND_TN ? (uint32_t)kt * BK * tc.A.ldb : (uint32_t)kt * (BK * 2);
    dma16(tc.A.r0, stage + q * 1024, tc.A.off[q0 & 1], soff + (uint32_t)q0 * tc.A.step);
  } else {
    char* dst = stage + B_OFF + q * 1024;
    if constexpr (KIND == KIND_TN) {
      dma16(tc.B.r0, dst, tc.B.off[q0 & 1], (uint32_t)kt * BK * tc.B.ldb + (uint32_t)q0 * tc.B.step);
    } else if constexpr (KIND == KIND_NN || KIND == KIND_NNS) {
      dma16(tc.B.r0, dst, tc.B.off[q0 & 1], ((uint32_t)kt * BK + (uint32_t)(q * 2)) * tc.B.ldb);
    } else if constexpr (KIND == KIND_FC1) {
      dma16((q0 & 1) ? tc.B.r1 : tc.B.r0, dst, tc.B.off[q0 & 1], (uint32_t)kt * (BK * 2) + (uint32_t)(q0 >> 1) * tc.B.step);
    } else {
      dma16(tc.B.r0, dst, tc.B.off[q0 & 1], (uint32_t)kt * (BK * 2) + (uint32_t)q0 * tc.B.step);
    }
  }
}

struct Frags {
  bf16x8_t a[FM], b[FN];
};

// The lane index recomputed where it is needed (two instructions) instead of
// kept in a register through the whole kernel.
__device__ __forceinline__ int lane_id() { return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// Per-lane byte offsets of the wave's fragments within an operand's region of
// a stage, computed once per tile so that a fragment read is one address
// addition plus an immediate offset.
//   K-contiguous operand: lane l reads row rb + l%16 (rb = 16 * fragment +
//   128 * wave row), chunk ks*4 + l/16; kc_swz(rb + l%16) = kc_swz(l%16), so
//   the offset is rb*128 + o[ks].
//   M/N-contiguous operand (256-wide, mn_swz): fragment n is columns
//   w*128 + 16n .. +15 (w: the wave's column); lane l (group g = l/16, i =
//   l%16) addresses k-row ks*32 + 8g + 4h + i/4 (h: which of the two
//   transposing reads) and columns 4(i%4) .. +3; mn_swz of that k-row is
//   4 ((i/4) % 4) ^ 2 (g % 2) whatever ks and h, so the offset is
//   o[n] + ks*16384 + h*2048.
template <bool MN>
struct Slots {
  int32_t o[MN ? FN : 2];
};

template <bool MN>
__device__ __forceinline__ void make_slots(Slots<MN>& sl, int w, int lane) {
  if constexpr (!MN) {
    const int r = lane & 15;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) sl.o[ks] = r * (BK * 2) + (((ks * 4 + (lane >> 4)) ^ kc_swz(r)) << 4);
  } else {
    const int g = lane >> 4, i = lane & 15;
    const int s = mn_swz(g * 8 + (i >> 2));
    const int base = (g * 8 + (i >> 2)) * (2 * BN) + (i & 1) * 8;
#pragma unroll
    for (int n = 0; n < FN; ++n) {
      const int c = w * 16 + n * 2 + ((i & 3) >> 1);
      sl.o[n] = base + ((c ^ s) << 4);
    }
  }
}

// Fragment (J-th of its operand) at a slot: K-contiguous rows rb .. rb+15;
// M/N-contiguous from two transposing reads (within each 16-lane group lane
// i receives column i of the 4 x 16 block the group addresses).
__device__ __forceinline__ bf16x8_t frag_kc(const char* t, int rb, int32_t o) {
  return *reinterpret_cast<const bf16x8_t*>(t + rb * (BK * 2) + o);
}
__device__ __forceinline__ bf16x8_t frag_mn(const char* t, int ks, int32_t o) {
  const char* p = t + ks * 32 * (2 * BN) + o;
  const bf16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_TR_PTR(p));
  const bf16x4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_TR_PTR(p + 4 * (2 * BN)));
  return bf16x8_t{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
}

template <int KIND>
struct TileSlots {
  Slots<a_is_mn<KIND>()> a;
  Slots<b_is_mn<KIND>()> b;
};

template <int KIND>
__device__ __forceinline__ TileSlots<KIND> tile_slots(int wm, int wn, int lane) {
  TileSlots<KIND> ts;
  make_slots(ts.a, wm, lane);
  make_slots(ts.b, wn, lane);
  return ts;
}

// Fragment J of k-step ks: A fragments 0 .. FM-1, then B fragments.
template <int KIND, int J>
__device__ __forceinline__ void read_frag(const char* stage, int ks, int wm, int wn, const TileSlots<KIND>& ts,
                                          Frags& f) {
  if constexpr (J < FM) {
    if constexpr (a_is_mn<KIND>()) f.a[J] = frag_mn(stage, ks, ts.a.o[J]);
    else f.a[J] = frag_kc(stage, wm * 128 + J * 16, ts.a.o[ks]);
  } else {
    if constexpr (b_is_mn<KIND>()) f.b[J - FM] = frag_mn(stage + B_OFF, ks, ts.b.o[J - FM]);
    else f.b[J - FM] = frag_kc(stage + B_OFF, wn * 128 + (J - FM) * 16, ts.b.o[ks]);
  }
}

// The I-th read of a k-step, in the order the (mt-major) MFMAs consume the
// fragments: A0, B0 .. B7, A1 .. A7.
constexpr int frag_order(int i) { return i == 0 ? 0 : i <= FN ? FM + i - 1 : i - FN; }

// MFMAs I .. I+N-1 of a k-step (index mt * FN + nt).  FIRST: from zero.  The
// B fragment goes first, so each accumulator holds its 16 x 16 output tile
// transposed: lane l holds output row l%16, columns 4*(l/16) .. +3.
template <int I, int N, bool FIRST = false>
__device__ __forceinline__ void mfma(const Frags& f, f32x4_t (&acc)[FM][FN]) {
#pragma unroll
  for (int x = I; x < I + N; ++x)
    acc[x / FN][x % FN] = mfma16(f.b[x % FN], f.a[x / FN], FIRST ? f32x4_t{} : acc[x / FN][x % FN]);
}

// Epilogue staging: a round is 64 of the wave's 128 rows; row r (0 .. 63) is
// 256 bytes (the wave's 128 columns) in 1 KB chunk (r/4) * NW + wave of the
// freed stage - the chunks this wave's own loads fill, so no other wave
// touches them - at offset (r%4) * 256, with 16-byte piece c at c ^ (r%16)
// (conflict-free 8-byte writes and 16-byte reads).
__device__ __forceinline__ int stg_off(int wave, int r, int c) {
  return ((r >> 2) * NW + wave) * 1024 + (r & 3) * 256 + ((c ^ (r & 15)) << 4);
}

// Stage tiles mt = 4*round .. +3, tiles nt = 0 .. NC-1 of the wave:
// v(mt, nt) returns the lane's four values (row l%16, columns 4*(l/16) .. +3
// of the tile) as four bf16; tile nt goes to the 16-column block blk(nt).
template <int NC, typename F, typename B>
__device__ __forceinline__ void stage_round(char* stage, int wave, int lane, int round, F v, B blk) {
  const int r16 = lane & 15, h = lane >> 4;
#pragma unroll
  for (int mtl = 0; mtl < 4; ++mtl) {
#pragma unroll
    for (int nt = 0; nt < NC; ++nt) {
      const int r = mtl * 16 + r16;
      const int x = blk(nt) * 32 + h * 8;  // byte of the 256-byte row
      *reinterpret_cast<uint2*>(stage + stg_off(wave, r, x >> 4) + (x & 15)) = v(4 * round + mtl, nt);
    }
    // one row of tiles at a time: the scheduler would otherwise read all of
    // the round's accumulators into VGPRs before the first write
    __builtin_amdgcn_sched_barrier(0);
  }
}

__device__ __forceinline__ uint4 staged(const char* stage, int wave, int r, int c) {
  return *reinterpret_cast<const uint4*>(stage + stg_off(wave, r, c));
}

__device__ __forceinline__ uint2 bf16x4(const f32x4_t& a) { return make_uint2(Elt::pack2(a[0], a[1]), Elt::pack2(a[2], a[3])); }

// Write out the wave's 128 x 128 share of a finished tile (two rounds of 64
// rows), with the kind's epilogue arithmetic - the same rounding points as
// grouped_gemm_kernel's epilogue.  Store q of a round covers 4 rows x 256
// bytes: lane l row q*4 + l/16, 16-byte piece l%16.
template <int KIND>
__device__ __forceinline__ void epilogue(const GemmParams& P, const TileInfo& ti, int wm, int wn, int wave, int lane,
                                         const f32x4_t (&acc)[FM][FN], char* stage) {
  asm volatile("" : "+v"(lane));
  const int cc = lane & 15, rq = lane >> 4;
  // Top-1 row map (KIND_NT, KIND_NN): the wave's 128 row targets (and the
  // rows' router weights) are loaded before the first store, since one
  // counter tracks this wave's loads and stores in issue order: lane l holds
  // those of rows l and 64 + l, and a store's lanes fetch theirs with a
  // cross-lane read.  Targets outside [0, M) are not written.
  const bool mapped = (KIND == KIND_NT || KIND == KIND_NN) && P.row_tok != nullptr;
  uint4 nns_g[KIND == KIND_NNS ? 2 : 1][4], nns_u[KIND == KIND_NNS ? 2 : 1][4];  // KIND_NNS: two quarters of gate/up
  int32_t tok2[2] = {-1, -1};
  uint32_t wt2[2] = {0, 0};
  if constexpr (KIND == KIND_NT || KIND == KIND_NN) {
    if (mapped) {
      const int64_t r0 = ti.row0 + wm * 128;
      const int32_t nrows = (int32_t)(ti.row_end - r0 < 0 ? 0 : (ti.row_end - r0 > 128 ? 128 : ti.row_end - r0));
      const __amdgpu_buffer_rsrc_t rt = make_rsrc(P.row_tok + r0, (uint64_t)nrows * 4);
      const __amdgpu_buffer_rsrc_t rw = make_rsrc(P.row_w + r0, (uint64_t)nrows * 2);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = h * 64 + lane;
        const int32_t tok = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rt, (uint32_t)r * 4u, 0, 0);
        tok2[h] = r < nrows ? tok : -1;
        if constexpr (KIND == KIND_NT) wt2[h] = __builtin_amdgcn_raw_buffer_load_b16(rw, (uint32_t)r * 2u, 0, 0);
      }
    }
  }
#pragma unroll
  for (int round = 0; round < 2; ++round) {
    // Rounds stay apart in the schedule: hoisting the next round's
    // accumulator reads and conversions would hold their registers.
    __builtin_amdgcn_sched_barrier(0);
    const int64_t rb = wm * 128 + round * 64;  // first tile row of the round
    if constexpr (KIND == KIND_FC1) {
      // The wave's 128 virtual columns: gate tiles nt = 0,1,4,5 and their up
      // tiles nt + 2, for intermediate columns jb .. jb+63.  Staged as
      // [gate 64 | up 64] (gu), then act = bf16(bf16(silu(gate)) * up).
      const int64_t I = P.I;
      const int64_t jb = (int64_t)ti.ntile * 128 + wn * 64;
      stage_round<FN>(stage, wave, lane, round, [&](int mt, int nt) { return bf16x4(acc[mt][nt]); },
                      [](int nt) { return ((nt & 2) ? 4 : 0) + (nt >> 2) * 2 + (nt & 1); });
      {
        const OutWin w = out_window(P.gu, ti.row0 + rb, ti.row_end, 2 * I);
        const int64_t j = jb + (cc & 7) * 8;
        const uint32_t voff = j < I ? (uint32_t)rq * w.rowb + (uint32_t)((cc < 8 ? 0 : I) + j) * 2u : kOOB;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          win_store(w, voff, q * 4, staged(stage, wave, q * 4 + rq, cc));
          if (q % 8 == 7) __builtin_amdgcn_sched_barrier(0);  // at most 8 staged reads in flight
        }
      }
      stage_round<4>(stage, wave, lane, round, [&](int mt, int k) {
        const int ng = (k >> 1) * 4 + (k & 1);
        float g[4], u[4];
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          g[e] = acc[mt][ng][e], g[e + 1] = acc[mt][ng][e + 1];
          u[e] = acc[mt][ng + 2][e], u[e + 1] = acc[mt][ng + 2][e + 1];
          Elt::round2(g[e], g[e + 1]);
          Elt::round2(u[e], u[e + 1]);
          g[e] = silu_f32(g[e]), g[e + 1] = silu_f32(g[e + 1]);
          Elt::round2(g[e], g[e + 1]);
        }
        return pack4(g[0] * u[0], g[1] * u[1], g[2] * u[2], g[3] * u[3]);
      }, [](int k) { return k; });
      {
        // act: 64 rows x 128 bytes; store q covers 8 rows, lane l row q*8 + l/8, piece l%8.
        const OutWin w = out_window(P.act, ti.row0 + rb, ti.row_end, I);
        const int c8 = lane & 7;
        const int64_t j = jb + c8 * 8;
        const uint32_t voff = j < I ? (uint32_t)(lane >> 3) * w.rowb + (uint32_t)j * 2u : kOOB;
#pragma unroll
        for (int q = 0; q < 8; ++q) win_store(w, voff, q * 8, staged(stage, wave, q * 8 + (lane >> 3), c8));
      }
    } else if constexpr (KIND == KIND_NNS) {
      // fc2 dgrad: the tile is dact (bf16, as the reference stores it) for
      // columns j < I; with the forward's gate/up of the same rows it becomes
      // [d_gate | d_up] of dG1.  The rows go in quarters of 16 (4 stores of
      // each half); each quarter's gate/up loads are issued a quarter ahead,
      // so that waiting for them does not also wait for the previous
      // quarter's stores (one counter tracks a wave's loads and stores in
      // issue order).  The next round's first loads go out during this
      // round's last quarter.
      const int64_t I = P.I;
      const int64_t j = (int64_t)ti.ntile * BN + wn * 128 + cc * 8;
      const uint32_t vg = j < I ? (uint32_t)rq * (uint32_t)(4 * I) + (uint32_t)j * 2u : kOOB;  // row rq of a quarter
      const uint32_t vu = vg + (uint32_t)I * 2u;
      // gate/up rows of quarter qq (0..7 over both rounds) of the wave's 128 rows
      auto window = [&](int qq) {
        return out_window(P.gin, ti.row0 + wm * 128 + (qq >> 2) * 64, ti.row_end, 2 * I);
      };
      auto load_q = [&](int qq, uint4 (&gv)[4], uint4 (&uv)[4]) __attribute__((always_inline)) {
        const OutWin wi = window(qq);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = (qq & 3) * 16 + q * 4;  // first row of the store within the round
          gv[q] = win_load(wi, vg, r);
          uv[q] = win_load(wi, vu, r);
        }
      };
      if (round == 0) load_q(0, nns_g[0], nns_u[0]);
      stage_round<FN>(stage, wave, lane, round, [&](int mt, int nt) { return bf16x4(acc[mt][nt]); },
                      [](int nt) { return nt; });
      const OutWin wo = out_window(P.c0, ti.row0 + rb, ti.row_end, 2 * I);
#pragma unroll
      for (int qr = 0; qr < 4; ++qr) {
        const int qq = round * 4 + qr;
        if (qq < 7) load_q(qq + 1, nns_g[(qq + 1) & 1], nns_u[(qq + 1) & 1]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = qr * 16 + q * 4;
          const uint4 v = staged(stage, wave, r + rq, cc);
          float d[8], g[8], u[8], dg[8], du[8];
          unpack8e<Elt>(v, d);
          unpack8e<Elt>(nns_g[qq & 1][q], g);
          unpack8e<Elt>(nns_u[qq & 1][q], u);
          swiglu_bwd8<Elt>(d, g, u, dg, du);
          win_store(wo, vg, r, pack8e<Elt>(dg));
          win_store(wo, vu, r, pack8e<Elt>(du));
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (KIND == KIND_TN) {
      // Rows m of copy g's gradient: those below csplit in c0, the rest in
      // c1 (split fc1), each tensor through a descriptor over the copy's rows
      // in it (the host sends a copy of more than 2 GiB to the 8-wave kernel).
      stage_round<FN>(stage, wave, lane, round, [&](int mt, int nt) { return bf16x4(acc[mt][nt]); },
                      [](int nt) { return nt; });
      const int64_t col = (int64_t)ti.ntile * BN + wn * 128 + cc * 8;
      const int64_t m0 = (int64_t)ti.mtile * BM + rb;  // first gradient row of the round
      const int64_t rows0 = P.csplit < P.M ? P.csplit : P.M;
      const OutWin w0 = {make_rsrc(P.c0 + ti.g * P.cgs, (uint64_t)rows0 * P.ldc * 2), (uint32_t)(P.ldc * 2)};
      const OutWin w1 = {make_rsrc(P.c1 + ti.g * P.cgs, (uint64_t)(P.M - rows0) * P.ldc * 2), (uint32_t)(P.ldc * 2)};
      const int64_t m = m0 + rq;  // the lane's row of store 0
      const bool cin = col < P.N;
      const bool split = uni(m0 + 63 >= rows0 ? 1 : 0) != 0;  // some row of the round lies in c1
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const uint4 v = staged(stage, wave, q * 4 + rq, cc);
        const int64_t mq = m + q * 4;
        const uint32_t o0 = cin && mq < rows0 ? (uint32_t)mq * w0.rowb + (uint32_t)col * 2u : kOOB;
        win_store(w0, o0, 0, v);
        if (split) {
          const uint32_t o1 = cin && mq >= rows0 ? (uint32_t)(mq - rows0) * w1.rowb + (uint32_t)col * 2u : kOOB;
          win_store(w1, o1, 0, v);
        }
        if (q % 8 == 7) __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      const int64_t col = (int64_t)ti.ntile * BN + wn * 128 + cc * 8;
      stage_round<FN>(stage, wave, lane, round, [&](int mt, int nt) { return bf16x4(acc[mt][nt]); },
                      [](int nt) { return nt; });
      const OutWin w = out_window(P.c0, ti.row0 + rb, ti.row_end, P.ldc);
      const uint32_t voff = col < P.N ? (uint32_t)rq * w.rowb + (uint32_t)col * 2u : kOOB;
      // Mapped rows go to row dst of the whole output (dst is -1 for rows
      // past the tile's group): through one descriptor over the output when
      // it spans at most 2 GiB, else through 64-bit addresses.
      const bool whole = (uint64_t)P.M * (uint64_t)P.ldc * 2u <= 0x7fffffffull;
      const OutWin wd = {make_rsrc(KIND == KIND_NT ? P.cout : P.c0, (uint64_t)P.M * P.ldc * 2), w.rowb};
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const uint4 v = staged(stage, wave, q * 4 + rq, cc);
        if (!(KIND == KIND_NN && mapped)) win_store(w, voff, q * 4, v);
        const int32_t d = mapped ? __shfl(tok2[round], q * 4 + rq, 64) : -1;
        const float wq = KIND == KIND_NT && mapped ? Elt::to_f32((uint32_t)__shfl((int32_t)wt2[round], q * 4 + rq, 64)) : 0.f;
        if ((KIND == KIND_NT || KIND == KIND_NN) && mapped && whole) {
          const uint32_t vd = col < P.N && (uint32_t)d < (uint32_t)P.M ? (uint32_t)d * wd.rowb + (uint32_t)col * 2u : kOOB;
          if (KIND == KIND_NN) {
            win_store(wd, vd, 0, v);
          } else {
            float f[8];
            unpack8e<Elt>(v, f);
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = __builtin_fmaf(f[e], wq, 0.f);
            win_store(wd, vd, 0, pack8e<Elt>(f));
          }
        } else if ((KIND == KIND_NT || KIND == KIND_NN) && mapped && col < P.N && (uint32_t)d < (uint32_t)P.M) {
          if (KIND == KIND_NN) {
            st_stream(P.c0 + (int64_t)d * P.ldc + col, v);
          } else {
            // the combine kernel's rounding: 0 + bf16(f * w), as fma(f, w, 0)
            float f[8];
            unpack8e<Elt>(v, f);
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = __builtin_fmaf(f[e], wq, 0.f);
            st_stream(P.cout + (int64_t)d * P.ldc + col, pack8e<Elt>(f));
          }
        }
        if (q % 8 == 7) __builtin_amdgcn_sched_barrier(0);
      }
    }
    // Keep each round's loads and stores in their round (register pressure).
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
}

// BAL (weight gradient): the balanced band order (build_wgrad_order); the
// host picks it when the grid is 8 XCDs x 32 blocks and G <= NT.
template <int KIND, bool BAL = false>
__global__ __launch_bounds__(NT, 1) void grouped_gemm_w4_kernel(GemmParams P) {
  static_assert(!BAL || KIND == KIND_TN, "the balanced order is the weight gradient's");
  __shared__ __attribute__((aligned(1024))) char lds[2 * STAGE_BYTES];
  __shared__ int32_t tpre[kMaxGroups + 1];
  __shared__ int32_t scan_buf[NT];
  __shared__ int4 ttab[kTileTab];
  const int t = threadIdx.x;
  const int wave = uni(t >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int G = P.G;

  const int64_t grid = gridDim.x;
  const int32_t xcd = (int32_t)(blockIdx.x % kNumXcd);
  const int32_t xj = (int32_t)(blockIdx.x / kNumXcd);
  int64_t ntn, tiles_per_group = 0, total;
  int32_t deal_rounds = 0;
  if constexpr (KIND == KIND_TN) {
    const int64_t mtn = (P.M + BM - 1) / BM;
    ntn = (P.N + BN - 1) / BN;
    tiles_per_group = mtn * ntn;
    total = tiles_per_group * G;
    if constexpr (BAL) {
      deal_rounds = uni(build_wgrad_order<NT>(P, tpre, scan_buf, t, total, tiles_per_group, xcd,
                                              reinterpret_cast<int32_t*>(lds), (int32_t)(sizeof(lds) / sizeof(int32_t))));
    }
  } else {
    ntn = (KIND == KIND_FC1) ? (P.I + 127) / 128 : (P.N + BN - 1) / BN;
    group_prefix<BM, NT>(P, tpre, scan_buf, t);
    total = (int64_t)tpre[G] * ntn;
  }
  int64_t slot = blockIdx.x;
  if ((grid & 7) == 0) slot = (blockIdx.x & 7) * (grid >> 3) + (blockIdx.x >> 3);
  const unsigned char* deal = reinterpret_cast<const unsigned char*>(tpre + G);

  // The block's first kTileTab tiles, decoded at once into LDS (see grouped_gemm_kernel).
  const int64_t rounds = (total + grid - 1) / grid;
  const int32_t ntab = (int32_t)(rounds < kTileTab ? rounds : kTileTab);
  const int32_t nk_all = KIND == KIND_TN ? 0 : (int32_t)((P.K + BK - 1) / BK);
  for (int e = t; e < ntab; e += NT) {
    TileInfo d;
    bool ok;
    if constexpr (!BAL) {
      const int64_t tile = slot + (int64_t)e * grid;
      ok = tile < total;
      if (ok) d = decode_tile<KIND, BM, false>(P, tile, tpre, G, ntn, tiles_per_group);
    } else {
      const int32_t x = e < deal_rounds ? (int32_t)deal[e] : ((e & 1) ? kNumXcd - 1 - xcd : xcd);
      const int64_t tile = ((int64_t)e * kNumXcd + x) * kBandTiles + xj;
      ok = tile < total;
      if (ok) {
        const int64_t rank = tile / tiles_per_group;
        d = decode_tile<KIND, BM, false>(P, scan_buf[rank], tpre, G, ntn, tiles_per_group, tile - rank * tiles_per_group);
      }
    }
    ttab[e] = ok ? make_int4(d.row0, d.row_end, d.g | (d.ntile << 12), d.mtile) : make_int4(0, 0, 0, -1);
  }
  __syncthreads();

  auto tile_at = [&](int64_t seq, TileInfo& ti) -> bool {
    if (seq < ntab) {
      const int4 e = ttab[seq];
      if (uni(e.w) < 0) return false;
      ti.row0 = uni(e.x);
      ti.row_end = uni(e.y);
      ti.g = uni(e.z) & 0xfff;
      ti.ntile = uni(e.z) >> 12;
      ti.mtile = uni(e.w);
      ti.nk = KIND == KIND_TN ? (int32_t)(((int64_t)ti.row_end - ti.row0 + BK - 1) / BK) : nk_all;
      return true;
    }
    if constexpr (!BAL) {
      const int64_t tile = slot + seq * grid;
      if (tile >= total) return false;
      ti = decode_tile<KIND, BM>(P, tile, tpre, G, ntn, tiles_per_group);
      return true;
    } else {
      const int32_t x = seq < deal_rounds ? uni((int32_t)deal[seq]) : ((seq & 1) ? kNumXcd - 1 - xcd : xcd);
      const int64_t tile = (seq * kNumXcd + x) * kBandTiles + xj;
      if (tile >= total) return false;
      const int64_t rank = tile / tiles_per_group;
      ti = decode_tile<KIND, BM>(P, uni(scan_buf[rank]), tpre, G, ntn, tiles_per_group, tile - rank * tiles_per_group);
      return true;
    }
  };

  // Consume cursor: the output tile being multiplied; tiles without K-tiles
  // (weight gradient of an empty group) are written as zeros on the way.
  int64_t c_seq = 0;
  TileInfo cur;
  for (;; ++c_seq) {
    if (!tile_at(c_seq, cur)) return;
    if (cur.nk > 0) break;
    zero_tile<BM, NT>(P, cur, t);
  }

  // Issue cursor: the stream K-tile whose loads go out next.  Past the
  // block's last K-tile it keeps its last tile with kt = 0, so those slots
  // re-load that tile's first K-tile (in bounds, never multiplied).
  Tile<KIND> it;
  int64_t i_seq = c_seq;
  int32_t i_kt = 0;
  bool i_live = true;
  it.i = cur;
  setup<KIND>(P, it, wave, lane_id());
  auto advance_issue = [&]() {
    if (!i_live) return;
    if (++i_kt < it.i.nk) return;
    i_kt = 0;
    while (tile_at(++i_seq, it.i)) {
      if (it.i.nk > 0) {
        setup<KIND>(P, it, wave, lane_id());
        return;
      }
    }
    i_live = false;
  };

  // Prologue: stream K-tiles 0 and 1 into the two stages; wait for the first.
  static_for<0, 2 * QO>([&](auto j) __attribute__((always_inline)) {
    issue<KIND, decltype(j)::value>(lds, it, i_kt, wave);
  });
  advance_issue();
  static_for<0, 2 * QO>([&](auto j) __attribute__((always_inline)) {
    issue<KIND, decltype(j)::value>(lds + STAGE_BYTES, it, i_kt, wave);
  });
  advance_issue();
  wait_loads<2 * QO>();
  block_barrier();
  int cs = 0;  // stage of the K-tile being multiplied
  f32x4_t acc[FM][FN];
  Frags f0, f1;
  {
    const TileSlots<KIND> ts = tile_slots<KIND>(wm, wn, lane_id());
    static_for<0, FM + FN>([&](auto j) __attribute__((always_inline)) {
      read_frag<KIND, frag_order(decltype(j)::value)>(lds, 0, wm, wn, ts, f0);
    });
  }

  // One k-step of MFMAs from `fm` (16 groups of 4), with the reads of k-step
  // KS of `stage` into `fr` and, with LOADS, load J0 + j of the next stream
  // K-tile into `refill` in the first 8 groups.
  // `ts` holds the wave's fragment offsets, computed once per tile from the
  // lane index passed through an opaque move, so that they are not hoisted
  // out of the tile loop, where they would hold registers during the epilogue.
  auto kstep = [&](auto ks, auto first, auto loads, auto j0, const char* stage, char* refill, const Frags& fm,
                   Frags& fr, const TileSlots<KIND>& ts) __attribute__((always_inline)) {
    static_for<0, 16>([&](auto jj) __attribute__((always_inline)) {
      constexpr int j = decltype(jj)::value;
      if constexpr (decltype(loads)::value == 2) issue<KIND, j>(refill, it, i_kt, wave);
      else if constexpr (decltype(loads)::value == 1 && j < QO) issue<KIND, decltype(j0)::value + j>(refill, it, i_kt, wave);
      if constexpr (decltype(ks)::value >= 0) read_frag<KIND, frag_order(j)>(stage, decltype(ks)::value, wm, wn, ts, fr);
      mfma<4 * j, 4, decltype(first)::value>(fm, acc);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  for (;;) {
    // Output tile `cur`.  Its first K-tile is in stage cs with k-step 0 in
    // f0; the next stream K-tile is in flight into the other stage.
    int ln = lane_id();
    asm volatile("" : "+v"(ln));
    const TileSlots<KIND> ts = tile_slots<KIND>(wm, wn, ln);
    kstep(Int<1>{}, Int<1>{}, Int<0>{}, Int<0>{}, lds + cs * STAGE_BYTES, nullptr, f0, f1, ts);
    wait_loads_lds<0>();
    block_barrier();
    cs ^= 1;
    for (int32_t kt = 1; kt < cur.nk; ++kt) {
      const char* stage = lds + cs * STAGE_BYTES;
      char* refill = lds + (cs ^ 1) * STAGE_BYTES;
      if constexpr ((PMX_W4_LOADS_FIRST_HALF >> KIND) & 1) {
        // all of the next K-tile's loads among the first k-step's MFMAs
        kstep(Int<0>{}, Int<0>{}, Int<2>{}, Int<0>{}, stage, refill, f1, f0, ts);
        kstep(Int<1>{}, Int<0>{}, Int<0>{}, Int<0>{}, stage, refill, f0, f1, ts);
      } else {
        // half of them in each k-step
        kstep(Int<0>{}, Int<0>{}, Int<1>{}, Int<0>{}, stage, refill, f1, f0, ts);
        kstep(Int<1>{}, Int<0>{}, Int<1>{}, Int<QO>{}, stage, refill, f0, f1, ts);
      }
      advance_issue();
      wait_loads_lds<0>();
      block_barrier();
      cs ^= 1;
    }
    // The tile's last k-step is in f1; stage cs holds the next stream
    // K-tile (published by the barrier) and stage cs ^ 1 is free.
    const TileInfo done = cur;
    bool more = false;
    while (tile_at(++c_seq, cur)) {
      if (cur.nk > 0) {
        more = true;
        break;
      }
      zero_tile<BM, NT>(P, cur, t);
    }
    mfma<0, FM * FN>(f1, acc);
    epilogue<KIND>(P, done, wm, wn, wave, lane_id(), acc, lds + (cs ^ 1) * STAGE_BYTES);
    if (!more) {
      wait_loads<0>();
      return;
    }
    // Once this wave's staging reads have returned, the next stream K-tile
    // goes into its chunks of the freed stage; then the next tile's first
    // k-step is read (after the epilogue, so that its 64 registers are free
    // during it).
    wait_lds();
    static_for<0, 2 * QO>([&](auto j) __attribute__((always_inline)) {
      issue<KIND, decltype(j)::value>(lds + (cs ^ 1) * STAGE_BYTES, it, i_kt, wave);
    });
    advance_issue();
    int ln2 = lane_id();
    asm volatile("" : "+v"(ln2));
    const TileSlots<KIND> ts2 = tile_slots<KIND>(wm, wn, ln2);
    static_for<0, FM + FN>([&](auto j) __attribute__((always_inline)) {
      read_frag<KIND, frag_order(decltype(j)::value)>(lds + cs * STAGE_BYTES, 0, wm, wn, ts2, f0);
    });
  }
}

}  // namespace w4

// Buffer offsets are 32-bit: one descriptor covers at most 2 GiB.
bool fits_rsrc(int64_t rows, int64_t ld) { return rows * ld * 2 < (int64_t)0x7fffffff; }

int g_num_cus = 0;

int grid_size() {
  if (g_num_cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -1;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
    g_num_cus = cus > 0 ? cus : 256;
  }
  return g_num_cus;
}

// 256 x 256 block tiles: a 64-deep K-tile (64 KB of operands) feeds 8.4
// MFLOP, half the bytes per flop of 128 x 256 tiles; operand delivery is what
// bounds this kernel, so that outweighs the coarser padding of ragged groups.
// Each wave's 128 x 64 share takes 128 accumulator registers per lane.
constexpr int kBM = 256;
constexpr int64_t kRsMaxRowsPerCopy = 8 * kBM;

// The four-wave kernel takes the calls of the kinds in PMX_W4_KINDS (bit
// KIND) whose loads can be FAST: fc1 + SwiGLU, fc2 dgrad + SwiGLU backward and
// the weight gradients, where it measured faster in the layer (config 3: fc1
// 3.02-3.05 vs 3.05 ms, fc2 dgrad 1.74-1.76 vs 1.73, fc2 wgrad 1.43 vs 1.48,
// fc1 wgrad 2.89-2.90 vs 2.93; Qwen3 shape: 0.81 vs 0.84, 0.49-0.50 vs 0.51,
// 0.46 vs 0.47, 0.78-0.79 vs 0.83).  The fc2 forward and the fc1 dgrad stay on
// the eight-wave kernel's register-staged loads, faster there (config 3: 1.65
// vs 1.67-1.68 and 3.06 vs 3.12-3.13; Qwen3 shape: 0.46 vs 0.50-0.51 and 0.80
// vs 0.85-0.86).  PMX_GEMM_W4=0 builds the eight-wave kernel for every call
// (the `w8` test variant, for comparisons).
#ifndef PMX_GEMM_W4
#define PMX_GEMM_W4 1
#endif
#ifndef PMX_W4_KINDS
#define PMX_W4_KINDS ((1 << KIND_FC1) | (1 << KIND_NNS) | (1 << KIND_TN))
#endif
template <int KIND>
constexpr bool use_w4() { return PMX_GEMM_W4 && ((PMX_W4_KINDS >> KIND) & 1); }

template <int KIND>
int launch(const GemmParams& P, hipStream_t stream) {
  // The LDS tile table keeps an n-tile index in 19 bits.
  const int64_t ntn = KIND == KIND_FC1 ? (P.I + 127) / 128 : (P.N + BN - 1) / BN;
  if (ntn >= (int64_t)1 << 19) return PMX_ERR_SHAPE;
  const int grid = grid_size();
  if (grid <= 0) return PMX_ERR_HIP;
  if constexpr (KIND == KIND_TN) {
    // FAST: every row of both operands within 31-bit offsets (P.K = their rows).
    const bool fast = fits_rsrc(P.K, P.M) && fits_rsrc(P.K, P.N);
    if constexpr (use_w4<KIND_TN>()) {
      if (fast && fits_rsrc(P.M, P.N)) {
        if (grid == kNumXcd * kBandTiles && P.G <= w4::NT) {
          w4::grouped_gemm_w4_kernel<KIND_TN, true><<<grid, w4::NT, 0, stream>>>(P);
        } else {
          w4::grouped_gemm_w4_kernel<KIND_TN><<<grid, w4::NT, 0, stream>>>(P);
        }
        PMX_LAUNCH_CHECK();
        return PMX_OK;
      }
    }
    const bool bal = grid == kNumXcd * kBandTiles && P.G <= NTHREADS;
    if (bal && fast) {
      grouped_gemm_kernel<KIND_TN, kBM, true, true><<<grid, NTHREADS, 0, stream>>>(P);
    } else if (bal) {
      grouped_gemm_kernel<KIND_TN, kBM, true><<<grid, NTHREADS, 0, stream>>>(P);
    } else if (fast) {
      grouped_gemm_kernel<KIND_TN, kBM, false, true><<<grid, NTHREADS, 0, stream>>>(P);
    } else {
      grouped_gemm_kernel<KIND_TN, kBM><<<grid, NTHREADS, 0, stream>>>(P);
    }
  } else {
    // FAST: K a multiple of 64, dgrad weights not split (P.b.split >= K).
    // RS (register-staged operands): fc1 and fc2 always; the fc1 dgrad when
    // the copies are small (under 8 m-tiles of rows on average), where each
    // weight strip serves few tiles and its loads wait on memory - with a
    // few large copies the DMA path is faster (it spends less power).
    const bool fast = P.K % BK == 0 && (KIND != KIND_NN || P.b.split >= P.K);
    if constexpr (use_w4<KIND>()) {
      if (fast) {
        w4::grouped_gemm_w4_kernel<KIND><<<grid, w4::NT, 0, stream>>>(P);
        PMX_LAUNCH_CHECK();
        return PMX_OK;
      }
    }
    if (!fast) {
      grouped_gemm_kernel<KIND, kBM><<<grid, NTHREADS, 0, stream>>>(P);
    } else if constexpr (KIND == KIND_FC1 || KIND == KIND_NT) {
      grouped_gemm_kernel<KIND, kBM, false, true, true><<<grid, NTHREADS, 0, stream>>>(P);
    } else if constexpr (KIND == KIND_NN) {
      if (P.M < kRsMaxRowsPerCopy * (int64_t)P.G) {
        grouped_gemm_kernel<KIND, kBM, false, true, true><<<grid, NTHREADS, 0, stream>>>(P);
      } else {
        grouped_gemm_kernel<KIND, kBM, false, true><<<grid, NTHREADS, 0, stream>>>(P);
      }
    } else {
      grouped_gemm_kernel<KIND, kBM, false, true><<<grid, NTHREADS, 0, stream>>>(P);
    }
  }
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

int PMX_GEMM_FN(pmx_gemm_fc1_swiglu_fwd)(const void* X, const void* w_gate, const void* w_up, int64_t w_copy_stride,
                            const int32_t* offsets, int32_t G, int64_t A, int64_t H, int64_t I, void* gu,
                            void* act, pmx_stream_t stream) {
  if (G <= 0 || G > kMaxGroups || A < 0 || H <= 0 || I <= 0) return PMX_ERR_ARG;
  if (H % 8 || I % 8 || A > INT32_MAX) return PMX_ERR_SHAPE;  // row offsets are int32
  if (A == 0) return PMX_OK;
  if (!X || !w_gate || !w_up || !offsets || !gu || !act) return PMX_ERR_ARG;
  if (!a16(X) || !a16(w_gate) || !a16(w_up)) return PMX_ERR_SHAPE;
  if (!fits_rsrc(I, H) || !fits_rsrc(kBM, H)) return PMX_ERR_SHAPE;
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

int PMX_GEMM_FN(pmx_group_gemm_nt)(const void* A, const void* B, const int32_t* offsets, int32_t G, int64_t M, int64_t N,
                      int64_t K, void* C, pmx_stream_t stream) {
  return PMX_GEMM_FN(pmx_group_gemm_nt_combine_top1)(A, B, offsets, G, M, N, K, C, nullptr, nullptr, nullptr, stream);
}

int PMX_GEMM_FN(pmx_group_gemm_nt_combine_top1)(const void* A, const void* B, const int32_t* offsets, int32_t G, int64_t M,
                                   int64_t N, int64_t K, void* C, const int32_t* row_token,
                                   const void* row_weight, void* out, pmx_stream_t stream) {
  if (G <= 0 || G > kMaxGroups || M < 0 || N <= 0 || K <= 0) return PMX_ERR_ARG;
  if (N % 8 || K % 8 || M > INT32_MAX) return PMX_ERR_SHAPE;  // row offsets are int32
  if (M == 0) return PMX_OK;
  if (!A || !B || !offsets || !C) return PMX_ERR_ARG;
  if (!a16(A) || !a16(B) || !a16(C)) return PMX_ERR_SHAPE;
  // the combine needs all three of its arguments, or none
  if ((row_token != nullptr) != (out != nullptr) || (row_token != nullptr) != (row_weight != nullptr)) {
    return PMX_ERR_ARG;
  }
  if (out && !a16(out)) return PMX_ERR_SHAPE;
  if (!fits_rsrc(N, K) || !fits_rsrc(kBM, K)) return PMX_ERR_SHAPE;
  GemmParams P = {};
  P.a = one(A, 0, K);
  P.b = one(B, N * K, K);
  P.offsets = offsets;
  P.G = G;
  P.M = M;
  P.N = N;
  P.K = K;
  P.c0 = static_cast<bf16_t*>(C);
  P.ldc = N;
  P.row_tok = row_token;
  P.row_w = static_cast<const bf16_t*>(row_weight);
  P.cout = static_cast<bf16_t*>(out);
  return launch<KIND_NT>(P, stream);
}

int PMX_GEMM_FN(pmx_group_gemm_nn)(const void* A, const void* B0, const void* B1, int64_t b_copy_stride, int64_t b_split,
                      const int32_t* offsets, int32_t G, int64_t M, int64_t N, int64_t K, void* C,
                      pmx_stream_t stream) {
  return PMX_GEMM_FN(pmx_group_gemm_nn_unpermute_top1)(A, B0, B1, b_copy_stride, b_split, offsets, G, M, N, K, nullptr, C,
                                          stream);
}

int PMX_GEMM_FN(pmx_group_gemm_nn_unpermute_top1)(const void* A, const void* B0, const void* B1, int64_t b_copy_stride,
                                     int64_t b_split, const int32_t* offsets, int32_t G, int64_t M, int64_t N,
                                     int64_t K, const int32_t* row_token, void* C, pmx_stream_t stream) {
  if (G <= 0 || G > kMaxGroups || M < 0 || N <= 0 || K <= 0) return PMX_ERR_ARG;
  if (N % 8 || K % 8 || M > INT32_MAX) return PMX_ERR_SHAPE;  // row offsets are int32
  if (M == 0) return PMX_OK;
  if (!A || !B0 || !offsets || !C) return PMX_ERR_ARG;
  if (!a16(A) || !a16(B0) || (B1 && !a16(B1)) || !a16(C)) return PMX_ERR_SHAPE;
  if (!fits_rsrc(K, N) || !fits_rsrc(kBM, K)) return PMX_ERR_SHAPE;
  GemmParams P = {};
  P.a = one(A, 0, K);
  P.b = one(B0, b_copy_stride, N);
  if (B1 != nullptr) {
    // one buffer->LDS instruction covers two k-rows of a 256-wide tile
    if (b_split <= 0 || b_split >= K || (b_split & 1)) return PMX_ERR_ARG;
    P.b.p1 = static_cast<const bf16_t*>(B1);
    P.b.split = b_split;
  }
  P.offsets = offsets;
  P.G = G;
  P.M = M;
  P.N = N;
  P.K = K;
  P.c0 = static_cast<bf16_t*>(C);
  P.ldc = N;
  P.row_tok = row_token;
  return launch<KIND_NN>(P, stream);
}

int PMX_GEMM_FN(pmx_gemm_fc2_dgrad_swiglu_bwd)(const void* dY, const void* w_down, const void* gu, const int32_t* offsets,
                                  int32_t G, int64_t A, int64_t H, int64_t I, void* dG1, pmx_stream_t stream) {
  if (G <= 0 || G > kMaxGroups || A < 0 || H <= 0 || I <= 0) return PMX_ERR_ARG;
  if (H % 8 || I % 8 || A > INT32_MAX) return PMX_ERR_SHAPE;  // row offsets are int32
  if (A == 0) return PMX_OK;
  if (!dY || !w_down || !gu || !offsets || !dG1) return PMX_ERR_ARG;
  if (!a16(dY) || !a16(w_down) || !a16(gu) || !a16(dG1)) return PMX_ERR_SHAPE;
  if (!fits_rsrc(H, I) || !fits_rsrc(kBM, H)) return PMX_ERR_SHAPE;
  // dact = dY @ Wdown[g], finished in the epilogue: dG1 = [d_gate | d_up].
  GemmParams P = {};
  P.a = one(dY, 0, H);
  P.b = one(w_down, H * I, I);
  P.offsets = offsets;
  P.G = G;
  P.N = I;
  P.K = H;
  P.I = I;
  P.c0 = static_cast<bf16_t*>(dG1);
  P.ldc = 2 * I;
  P.gin = static_cast<const bf16_t*>(gu);
  return launch<KIND_NNS>(P, stream);
}

int PMX_GEMM_FN(pmx_group_gemm_tn)(const void* A, const void* B, const int32_t* offsets, int32_t G, int64_t K, int64_t M,
                      int64_t N, void* C0, void* C1, int64_t c_copy_stride, int64_t c_split, pmx_stream_t stream) {
  if (G <= 0 || G > kMaxGroups || K < 0 || M <= 0 || N <= 0) return PMX_ERR_ARG;
  if (M % 8 || N % 8) return PMX_ERR_SHAPE;
  // One K-tile (64 rows) of either operand lies within one descriptor; the
  // group as a whole may span any number of bytes (rebased per K-tile).
  if (!fits_rsrc(BK, M) || !fits_rsrc(BK, N)) return PMX_ERR_SHAPE;
  if (!A || !B || !offsets || !C0) return PMX_ERR_ARG;
  if (C1 && (c_split <= 0 || c_split >= M)) return PMX_ERR_ARG;
  // 16-byte row segments of C: both tensors aligned, copies 8-element aligned
  // and apart by at least the rows each tensor holds (no two copies overlap).
  if (!a16(A) || !a16(B) || !a16(C0) || (C1 && !a16(C1)) || c_copy_stride % 8) return PMX_ERR_SHAPE;
  const int64_t c_rows = C1 ? (c_split > M - c_split ? c_split : M - c_split) : M;
  if (G > 1 && c_copy_stride < c_rows * N) return PMX_ERR_ARG;
  GemmParams P = {};
  P.a = one(A, 0, M);
  P.b = one(B, 0, N);
  P.offsets = offsets;
  P.G = G;
  P.K = K;
  P.M = M;
  P.N = N;
  P.c0 = static_cast<bf16_t*>(C0);
  P.c1 = C1 ? static_cast<bf16_t*>(C1) : static_cast<bf16_t*>(C0);
  P.cgs = c_copy_stride;
  P.ldc = N;
  P.csplit = C1 ? c_split : INT64_MAX;
  return launch<KIND_TN>(P, stream);
}

}  // extern "C"
