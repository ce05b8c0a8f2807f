/*
 * placemoe_amd.h - C ABI of the MI355X (gfx950) PlaceMoE expert-layer library.
 *
 * One GPU's share of the PlaceMoE / VeOmni MoE expert layer:
 *   map (M table) -> histogram/scan -> permute -> SwiGLU grouped GEMM
 *   (fwd, dgrad, wgrad) -> router-weighted combine -> replica-gradient fold.
 *
 * Conventions
 *  - Every entry point returns PMX_OK (0) or a PMX_ERR_* code; nothing throws.
 *  - All pointers are device pointers; every buffer, including workspace, is
 *    allocated by the caller.  The library allocates nothing, never
 *    synchronises the host, and enqueues work only on the given stream.
 *  - bf16 tensors are passed as `const void*` holding bf16 bit patterns,
 *    row-major and contiguous (fp16 tensors go to the *_f16 entry points,
 *    see "fp16 tensors" at the end).  Index tensors are int32 unless stated.
 *  - Positions, row offsets and the row kernels' token rows are 32-bit:
 *    assignments T*K, GEMM row counts and segment-sum rows above 2^31-1
 *    return PMX_ERR_SHAPE before anything is launched.
 *  - Each declaration names the reference (pia7a/PlaceMoE) interface it
 *    replaces, as `file:line`.
 */
#ifndef PLACEMOE_AMD_H
#define PLACEMOE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* pmx_stream_t; /* == hipStream_t */

#define PMX_OK 0
#define PMX_ERR_HIP 1      /* a HIP runtime call or kernel launch failed */
#define PMX_ERR_ARG 2      /* bad argument: null pointer, negative size, K too large */
#define PMX_ERR_SHAPE 3    /* shape the kernels do not support (e.g. dim not a multiple of 8) */
#define PMX_ERR_RANGE 4    /* device check found an index outside its table (routing status word) */

/* Library identification and error text. */
const char* pmx_version(void);
const char* pmx_error_string(int code);

/* ------------------------------------------------------------------------ */
/* Routing: map -> histogram -> scan -> stable scatter index                */
/* ------------------------------------------------------------------------ */

/* Bytes of workspace pmx_route needs for `num_assign` assignments over
 * `num_slots` physical copies.  The first 16 bytes of the workspace hold the
 * routing status word read by pmx_route_status. */
size_t pmx_route_workspace_bytes(int64_t num_assign, int32_t num_slots);

/* Full integer routing path, bit-exact with the reference:
 *   phys[t,k]  = M[src[t], sel[t,k]]                (M table gather)
 *   counts[c]  = #{(t,k) : phys[t,k] == c}           (histogram)
 *   offsets[c] = sum_{c'<c} counts[c'], offsets[C] = T*K
 *   pos[t,k]   = offsets[phys[t,k]] + #{a' < t*K+k : phys[a'] == phys[t,k]}
 * i.e. pos = phys.flatten().argsort(stable=True).argsort().
 * Replaces ExpertSwapManager.map_logical_to_physical
 *   (veomni/distributed/moe/hiermoe/expert_swap.py:5831-5879, source LUT
 *   gather at :5914-5921), expert_histogram
 *   (veomni/ops/kernels/moe/_kernels/kernel/moe.py:53-82), the cumsum and
 *   double argsort of MergedFc1TritonFusedMoeExpertFunction.forward
 *   (veomni/ops/kernels/moe/group_gemm.py:473-477) and
 *   _local_expert_sort_indices (veomni/distributed/moe/hiermoe/all_to_all.py:820-847).
 * sel: int64 [T*K] logical expert ids.  M: int64 [S*E] (row s = source s), or
 *   NULL for the identity map (phys = sel, then E must equal C).
 * src: int64 [T] source ids, or NULL to use `src_const` for every token.
 * Out-of-range ids are clamped and flagged in the status word. */
int pmx_route(const int64_t* sel, const int64_t* M, const int64_t* src, int32_t src_const,
              int32_t S, int32_t E, int64_t T, int32_t K, int32_t C,
              int32_t* phys, int32_t* counts, int32_t* offsets, int32_t* pos,
              void* workspace, size_t workspace_bytes, pmx_stream_t stream);

/* Allocation-free variant of pmx_route, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It has no counterpart in the reference.  Same kernels and
 * results as pmx_route; the chunk table lives in a static device array of
 * 8 MiB per GPU (held until the process ends) instead of a caller workspace,
 * and the routing status word (0 = every index valid) is written to
 * `status` (device int32; NULL drops it).  Calls no allocating routine.
 * Limit: pmx_route_workspace_bytes(T*K, C) must not exceed 8 MiB (every T
 * when C <= 2000), else PMX_ERR_SHAPE before anything is launched.  Calls
 * on one GPU share the array: calls that overlap on one GPU (different
 * streams, or threads) race; calls ordered on one stream do not. */
int pmx_route_noalloc(const int64_t* sel, const int64_t* M, const int64_t* src, int32_t src_const,
                      int32_t S, int32_t E, int64_t T, int32_t K, int32_t C,
                      int32_t* phys, int32_t* counts, int32_t* offsets, int32_t* pos,
                      int32_t* status, pmx_stream_t stream);

/* Copies the routing status word (0 = all indices valid) to host memory;
 * synchronises `stream`.  For tests and debug validation only. */
int pmx_route_status(const void* workspace, int32_t* status_host, pmx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Row movement                                                              */
/* ------------------------------------------------------------------------ */

/* Xp[pos[t,k]] = X[t] for every k.  X [T,H] bf16 -> Xp [T*K,H] bf16.
 * Replaces moe_scatter (veomni/ops/kernels/moe/_kernels/kernel/moe.py:299-333). */
int pmx_moe_scatter(const void* X, const int32_t* pos, int64_t T, int32_t K, int64_t H,
                    void* Xp, pmx_stream_t stream);

/* pmx_moe_scatter that also records where each row came from:
 * row_src[pos[t,k]] = t*K + k (int32 [T*K]; NULL: not written) and, given
 * the router weights w (bf16 [T,K]), each row's weight row_w[pos[t,k]] =
 * w[t,k] (bf16 [T*K]; w and row_w both given or both NULL, and only with
 * row_src).  With top-1 routing (K = 1) row_src[r] is the token of row r:
 * the row map of pmx_group_gemm_nt_combine_top1 and
 * pmx_group_gemm_nn_unpermute_top1; the call then writes the map first and
 * copies the rows in their storage order (a row that pos does not name gets
 * row_src -1 and a zero row, its row_w is left as it was; pos from pmx_route
 * names every row).  Replaces moe_scatter (moe.py:299-333)
 * plus the inverse of the scatter index that moe_gather's backward reads
 * (moe.py:126-159). */
int pmx_moe_scatter_src(const void* X, const int32_t* pos, const void* w, int64_t T, int32_t K,
                        int64_t H, void* Xp, int32_t* row_src, void* row_w, pmx_stream_t stream);

/* out[t] = bf16( sum_k fp32(Y[pos[t,k]]) ).  Y [T*K,H] bf16 -> out [T,H] bf16.
 * Replaces moe_gather (veomni/ops/kernels/moe/_kernels/kernel/moe.py:126-159). */
int pmx_moe_gather(const void* Y, const int32_t* pos, int64_t T, int32_t K, int64_t H,
                   void* out, pmx_stream_t stream);

/* Router-weighted combine:
 *   out[t] = bf16( sum_k fp32( bf16(Y[pos[t,k]] * w[t,k]) ) ),  w: bf16 [T,K].
 * Replaces rank_dedup_combine (veomni/distributed/moe/hiermoe/all_to_all.py:2539-2564)
 * with its fp32 segment sum (_aggregate_weighted_outputs :2266-2294,
 * segment_sum_dim0_fp32_to_source_dtype triton_segment_sum.py:52-103) on one rank. */
int pmx_combine_fwd(const void* Y, const int32_t* pos, const void* w, int64_t T, int32_t K,
                    int64_t H, void* out, pmx_stream_t stream);

/* Gradient of pmx_combine_fwd:
 *   dY[pos[t,k]] = bf16(dout[t] * w[t,k])
 *   dw[t,k]      = bf16( sum_h fp32( bf16(dout[t,h] * Y[pos[t,k],h]) ) )
 * Replaces the autograd of the weighted multiply in rank_dedup_combine
 * (all_to_all.py:2552) and _CudaIndexAddDim0CastOutput.backward (:930-933). */
int pmx_combine_bwd(const void* dout, const void* Y, const int32_t* pos, const void* w,
                    int64_t T, int32_t K, int64_t H, void* dY, void* dw, pmx_stream_t stream);

/* Top-1 routing only (K = 1): pmx_combine_bwd walked in the rows' storage
 * order.  Row r of Y and dY belongs to token row_token[r] (the row map that
 * pmx_moe_scatter_src writes), so Y is read and dY written front to back and
 * only dout is gathered:
 *   dY[r]            = bf16(dout[row_token[r]] * w[row_token[r]])
 *   dw[row_token[r]] = bf16( sum_h fp32( bf16(dout[row_token[r],h] * Y[r,h]) ) )
 * Bit-identical to pmx_combine_bwd(dout, Y, pos, w, T, 1, H, dY, dw) when
 * row_token is the row map of pos.  A row whose row_token lies outside
 * [0, T) gets dY[r] = 0 and writes no dw.  H must be a multiple of 8 and
 * dout, Y, dY 16-byte aligned (PMX_ERR_SHAPE otherwise).  Replaces the same
 * reference code as pmx_combine_bwd (all_to_all.py:2552, :930-933). */
int pmx_combine_bwd_top1_rows(const void* dout, const void* Y, const int32_t* row_token, const void* w,
                              int64_t T, int64_t H, void* dY, void* dw, pmx_stream_t stream);

/* Bytes of workspace pmx_segment_sum needs. */
size_t pmx_segment_sum_workspace_bytes(int64_t num_src_rows, int64_t num_rows);

/* out[r] = sum_{i : index[i]==r} source[i] in fp32, stored as bf16.
 * index: int64 [N]; rows are summed in ascending i (stable) order.
 * Replaces segment_sum_dim0_fp32_to_source_dtype
 * (veomni/distributed/moe/hiermoe/triton_segment_sum.py:52-103). */
int pmx_segment_sum(const void* source, const int64_t* index, int64_t N, int64_t H,
                    int64_t num_rows, void* out, void* workspace, size_t workspace_bytes,
                    pmx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* SwiGLU grouped GEMM over per-copy row groups                              */
/* ------------------------------------------------------------------------ */
/* Group g owns rows [offsets[g], offsets[g+1]) of the permuted activations;
 * offsets is the int32 [G+1] array produced by pmx_route (device memory).
 * Weights of copy g: gate rows at w_gate + g*w_copy_stride, up rows at
 * w_up + g*w_copy_stride, each [I, H] row-major.  A merged gate_up_proj
 * [G, 2I, H] is w_gate = W, w_up = W + I*H, w_copy_stride = 2*I*H; split
 * fc1_1/fc1_2 weights [G, I, H] use w_copy_stride = I*H.
 * 1 <= G <= 2048; H, I, N and K must be multiples of 8 and every tensor
 * 16-byte aligned (PMX_ERR_SHAPE otherwise). */

/* Forward fc1 with the SwiGLU epilogue:
 *   gu[a, 0:I] = bf16(X[a] @ Wgate[g]^T), gu[a, I:2I] = bf16(X[a] @ Wup[g]^T)
 *   act[a]     = bf16( bf16(silu(gate)) * up )
 * X [A,H], gu [A,2I], act [A,I].  Replaces the fc1 group_gemm_same_nk +
 * chunk + silu + multiply of EPMergedFc1GroupGemm.forward
 * (veomni/distributed/moe/moe_layer.py:376-397) and EPGroupGemm.forward (:167-193). */
int pmx_gemm_fc1_swiglu_fwd(const void* X, const void* w_gate, const void* w_up,
                            int64_t w_copy_stride, const int32_t* offsets, int32_t G,
                            int64_t A, int64_t H, int64_t I, void* gu, void* act,
                            pmx_stream_t stream);

/* Ragged-M grouped GEMM, B transposed: C[a] = bf16(A[a] @ B[g]^T), B [G,N,K].
 * Forward fc2 (A = act, B = down_proj [G,H,I]).
 * Replaces group_gemm_same_nk(transpose_b=True)
 * (veomni/ops/kernels/moe/_kernels/kernel/group_gemm.py:170-247). */
int pmx_group_gemm_nt(const void* A, const void* B, const int32_t* offsets, int32_t G,
                      int64_t M, int64_t N, int64_t K, void* C, pmx_stream_t stream);

/* Top-1 routing only (K = 1: every token has exactly one row): pmx_group_gemm_nt
 * with the router-weighted combine in its epilogue.  Writes C [M,N] as
 * pmx_group_gemm_nt does and out[row_token[r]] = bf16(0 + bf16(C[r] * row_weight[r]))
 * (out [M,N], row_weight bf16 [M]: the router weight of row r), bit-identical
 * to pmx_combine_fwd(C, pos, w, M, 1, N, out) when row_token and row_weight
 * are the row map of pos and w (pmx_moe_scatter_src).  Rows whose row_token
 * lies outside [0, M) are not combined.  row_token, row_weight and out are all
 * given or all NULL (NULL: pmx_group_gemm_nt).  Replaces
 * group_gemm_same_nk(transpose_b=True) (group_gemm.py:170-247) followed by
 * rank_dedup_combine (all_to_all.py:2539-2564) for a top-1 layer. */
int pmx_group_gemm_nt_combine_top1(const void* A, const void* B, const int32_t* offsets,
                                   int32_t G, int64_t M, int64_t N, int64_t K, void* C,
                                   const int32_t* row_token, const void* row_weight, void* out,
                                   pmx_stream_t stream);

/* Ragged-M grouped GEMM, B not transposed: C[a] = bf16(A[a] @ B[g]), B [G,K,N];
 * B rows k >= b_split come from B1 (for split fc1 weights), else from B0;
 * pass B1 = NULL for a single tensor.  dgrad fc1 (A = dG1 [A,2I]).
 * Replaces group_gemm_same_nk(transpose_b=False) (group_gemm.py:170-247). */
int pmx_group_gemm_nn(const void* A, const void* B0, const void* B1, int64_t b_copy_stride,
                      int64_t b_split, const int32_t* offsets, int32_t G, int64_t M,
                      int64_t N, int64_t K, void* C, pmx_stream_t stream);

/* Top-1 routing only: pmx_group_gemm_nn whose output row r is written to row
 * row_token[r] of C [M,N] (NULL: row r, as pmx_group_gemm_nn).  With row_token
 * the inverse of pos this is the unpermute gradient of a top-1 layer,
 * bit-identical to pmx_group_gemm_nn followed by pmx_moe_gather(.., K = 1, ..).
 * Rows whose row_token lies outside [0, M) are not written.  Replaces
 * group_gemm_same_nk(transpose_b=False) (group_gemm.py:170-247) followed by
 * moe_gather (moe.py:126-159) for a top-1 layer. */
int pmx_group_gemm_nn_unpermute_top1(const void* A, const void* B0, const void* B1,
                                     int64_t b_copy_stride, int64_t b_split,
                                     const int32_t* offsets, int32_t G, int64_t M, int64_t N,
                                     int64_t K, const int32_t* row_token, void* C,
                                     pmx_stream_t stream);

/* dgrad fc2 followed by the SwiGLU backward:
 *   dact = bf16(dY[a] @ down[g])                      ([A,I])
 *   dG1[a, 0:I] = d_gate, dG1[a, I:2I] = d_up         (silu_backward rounding)
 * dY [A,H], down [G,H,I], gu [A,2I] from the forward, dG1 [A,2I].  One
 * launch on `stream`: the GEMM's epilogue rounds dact to bf16, reads the
 * rows' gate/up and writes both halves of dG1 (no workspace; dact is never
 * stored).
 * Replaces the dgrad + silu_backward + cat of EPMergedFc1GroupGemm.backward
 * (veomni/distributed/moe/moe_layer.py:453-482). */
int pmx_gemm_fc2_dgrad_swiglu_bwd(const void* dY, const void* w_down, const void* gu,
                                  const int32_t* offsets, int32_t G, int64_t A, int64_t H,
                                  int64_t I, void* dG1, pmx_stream_t stream);

/* Ragged-K grouped GEMM (weight gradient):
 *   C[g] = bf16(A[rows of g]^T @ B[rows of g]),  A [K,M], B [K,N], C [G,M,N],
 * K = the rows of A and B (offsets[G] <= K); it selects the addressing: up to
 * 2 GiB per operand, one descriptor per group; beyond, 64-bit windows rebased
 * per 64-row K-tile (any group size);
 * a group with no rows stores zeros.  Rows m >= c_split of C[g] go to C1
 * (split fc1 gradients, row m - c_split), else to C0; pass C1 = NULL for one
 * tensor.  Copy g of either tensor starts c_copy_stride elements after copy
 * g - 1 (a multiple of 8, at least the rows the tensor holds times N); A, B,
 * C0 and C1 are 16-byte aligned (PMX_ERR_SHAPE / PMX_ERR_ARG otherwise).
 * A and B must be valid device pointers even when every group is empty
 * (PMX_ERR_ARG otherwise); with no rows at all the caller can skip the call,
 * since every C[g] is zero.
 * Replaces group_gemm_same_mn(transpose_a=True)
 * (veomni/ops/kernels/moe/_kernels/kernel/group_gemm.py:370-410). */
int pmx_group_gemm_tn(const void* A, const void* B, const int32_t* offsets, int32_t G,
                      int64_t K, int64_t M, int64_t N, void* C0, void* C1,
                      int64_t c_copy_stride, int64_t c_split, pmx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Router weight on the fc2 input (the reference's non-EP arithmetic)        */
/* ------------------------------------------------------------------------ */

/* out[r] = bf16(act[r] * row_w[r]);  act, out [R,N] bf16, row_w bf16 [R]
 * (each permuted row's router weight, as pmx_moe_scatter_src writes it).
 * Replaces fc1_weighted_output = fc1_activation * scattered_gate_weight
 * (veomni/ops/kernels/moe/group_gemm.py:269-276 split, :494-499 merged). */
int pmx_weight_rows(const void* act, const void* row_w, int64_t R, int64_t N, void* out,
                    pmx_stream_t stream);

/* Backward of pmx_weight_rows fused with the SwiGLU backward, per row r:
 *   dact          = bf16(d_act_w[r] * row_w[r])
 *   dw[row_src[r]] = bf16( sum_j fp32( bf16(act[r,j] * d_act_w[r,j]) ) )
 *   dG1[r]        = [ d_gate | d_up ] of dact with the rounding points of
 *                   pmx_gemm_fc2_dgrad_swiglu_bwd (aten silu_backward)
 * d_act_w, act [R,I], gu and dG1 [R,2I] (gate | up) bf16; row_src int32 [R]
 * (the row's index t*K+k in dw [A] bf16; entries outside [0, A) write no dw;
 * row_src and dw both NULL: no dw).  Replaces group_gemm.py:365-377 and :406
 * (split), :577-592 (merged). */
int pmx_swiglu_bwd_weighted(const void* d_act_w, const void* gu, const void* act, const void* row_w,
                            const int32_t* row_src, int64_t R, int64_t I, int64_t A, void* dG1,
                            void* dw, pmx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Replica-gradient fold                                                     */
/* ------------------------------------------------------------------------ */

/* out[e, p] = sum over copies c of e (copy_slots[copy_offsets[e] .. copy_offsets[e+1]),
 *             slot order) with slot_tokens[c] > 0 of fp32(grads[c, p]).
 * grads: bf16 [C,P]; out: fp32 [E,P]; slot_tokens: int64 [C] tokens seen by
 * each copy, or NULL to treat every copy as active.  If writeback != 0 every
 * copy of e (active or not) is overwritten with bf16(out[e]).
 * A copy_slots entry outside [0, C) is neither read nor written and sets
 * *status (device int32, caller-zeroed; may be NULL) to 1.
 * Replaces _zero_inactive_slot_grads_for_layer (expert_swap.py:6250-6262),
 * _replica_grad_contributions (:6839-6876) and _unpack_replica_grad
 * (:6886-6889) for the copies held by one GPU. */
int pmx_replica_fold(void* grads, const int32_t* copy_offsets, const int32_t* copy_slots,
                     const int64_t* slot_tokens, int32_t E, int32_t C, int64_t P, float* out,
                     int32_t writeback, int32_t* status, pmx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Cross-rank replica-gradient exchange: the per-rank halves                 */
/* ------------------------------------------------------------------------ */

/* Gradient element types of the exchange entry points. */
#define PMX_DTYPE_BF16 0
#define PMX_DTYPE_F32 1
#define PMX_DTYPE_F16 2

/* An exchange item is one logical expert x one parameter.  grads: [C, P]
 * copy gradients of this rank (`dtype`), item i's local copies are
 * slots[slot_offsets[i] .. slot_offsets[i+1]).  Pointer lists hold device
 * addresses (int64) of P-element regions: item i's outputs are
 * out_ptrs[out_offsets[i] .. out_offsets[i+1]), its received parts
 * part_ptrs[part_offsets[i] .. part_offsets[i+1]).  Sums accumulate in fp32
 * (local slots in list order, then parts in list order) and are stored once
 * in `dtype`.  A slot outside [0, C) is skipped and sets *status to 1.
 *
 * pack:   out = sum of the item's local copies, written to each output
 *         region (the send buffers).  Replaces the local sums of
 *         _replica_grad_contributions (expert_swap.py:6839-6876) and
 *         _pack_replica_grad_items (:6907-6929).
 * unpack: total = (with_local ? sum of local copies : 0) + sum of parts,
 *         written into every local copy and to each output region (an
 *         owner's broadcast buffers; out lists may be NULL).  Replaces the
 *         receive halves of _sync_pairwise_replica_gradients (:7038-7107:
 *         local_sum + remote), _sync_owner_replica_gradients (:7109-7217:
 *         owner total and broadcast) and _unpack_replica_grad (:6886-6889).
 * The transfer between ranks (RCCL send/recv or all-to-all) is the caller's. */
int pmx_replica_exchange_pack(const void* grads, int32_t dtype, int64_t P, int32_t C, int32_t n_items,
                              const int32_t* slot_offsets, const int32_t* slots, const int32_t* out_offsets,
                              const int64_t* out_ptrs, int32_t* status, pmx_stream_t stream);
int pmx_replica_exchange_unpack(void* grads, int32_t dtype, int64_t P, int32_t C, int32_t n_items,
                                const int32_t* slot_offsets, const int32_t* slots, int32_t with_local,
                                const int32_t* part_offsets, const int64_t* part_ptrs, const int32_t* out_offsets,
                                const int64_t* out_ptrs, int32_t* status, pmx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Route statistics for the placement planner                               */
/* ------------------------------------------------------------------------ */

/* Source-conditioned demand and co-selection counts of one routing sample,
 * added to caller-zeroed int64 tables (so a profiling window accumulates on
 * the device):
 *   demand[s,e]     += #{(t,k) : src(t) == s, sel[t,k] == e}
 *   affinity[s,a,b] += #{(t, k < k') : src(t) == s, {sel[t,k], sel[t,k']} == {a,b}}, a != b
 * (symmetric, zero diagonal).  sel: int64 [T*K] logical expert ids; src:
 * int64 [T] source ranks, or NULL for `src_const`; demand [S*E]; affinity
 * [S*E*E]; K <= 32.  A token with an id outside [0,E) or a source outside
 * [0,S) is skipped and sets *status (device int32, caller-zeroed) to 1.
 * Replaces profile_route_statistics
 * (veomni/distributed/moe/hiermoe/placemoe/statistics.py:30-64). */
int pmx_route_statistics(const int64_t* sel, const int64_t* src, int32_t src_const, int32_t S,
                         int32_t E, int64_t T, int32_t K, int64_t* demand, int64_t* affinity,
                         int32_t* status, pmx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Expert-parallel payloads (the per-rank halves around the all-to-all)     */
/* ------------------------------------------------------------------------ */

/* Bytes of workspace pmx_ep_dispatch_payload needs. */
size_t pmx_ep_payload_workspace_bytes(int64_t num_assign, int32_t num_ranks);

/* Rank-deduplicated dispatch payload of one EP rank.  Assignment (t,k) with
 * physical slot phys[t,k] goes to rank r = phys / slots_per_rank; a token's
 * hidden row is sent once per distinct target rank.
 *   assign_counts[r], assign_offsets[R+1]: assignments per target rank
 *       (assignment_send_splits) and their exclusive prefix;
 *   unique_counts[r], unique_offsets[R+1]: distinct (rank, token) pairs per
 *       rank (unique_send_splits); U = unique_offsets[R];
 *   send_hidden [U,H] bf16 (capacity T*K rows): row u = hidden[unique_tokens[u]],
 *       pairs ordered by (rank, token);
 *   unique_tokens [U] int32 (local_unique_token_indices);
 *   send_meta [T*K,3] int32: (ordinal of the assignment's pair within its
 *       rank, local slot, token) with assignments ordered by (rank, token, k);
 *   send_weights [T*K] bf16: the routing weight of each, same order;
 *   target_rank [T*K] int32 in (t,k) order.
 * Ties within one (rank, token) pair keep k order (the reference sorts the
 * keys with an unstable argsort, which leaves that order open).  phys: int32
 * [T*K]; weights: bf16 [T*K]; hidden: bf16 [T,H], H % 8 == 0; K <= 32.  A
 * slot outside [0, R*slots_per_rank) is clamped and sets *status (device
 * int32, caller-zeroed) to 1.
 * Replaces _build_local_payload
 * (veomni/distributed/moe/hiermoe/all_to_all.py:979-1055). */
int pmx_ep_dispatch_payload(const int32_t* phys, const void* hidden, const void* weights, int64_t T,
                            int32_t K, int64_t H, int32_t R, int32_t slots_per_rank,
                            int32_t* assign_counts, int32_t* assign_offsets, int32_t* unique_counts,
                            int32_t* unique_offsets, void* send_hidden, int32_t* unique_tokens,
                            int32_t* send_meta, void* send_weights, int32_t* target_rank,
                            int32_t* status, void* workspace, size_t workspace_bytes,
                            pmx_stream_t stream);

/* Bytes of workspace pmx_ep_combine_aggregate needs for `num_recv` received
 * assignments. */
size_t pmx_ep_combine_workspace_bytes(int64_t num_recv);

/* Combine on the rank that ran the experts: the weighted outputs of its N
 * received assignments (receive order: source-rank major, tokens ascending
 * within each source), summed in fp32 per run of equal (src_rank, src_token):
 *   out[u] = bf16( sum_{a in run u} fp32( bf16(Y[pos[a]] * w[a]) ) ),
 * where Y [*,H] bf16 holds the expert outputs in expert order and pos[a] is
 * the row of assignment a in Y.  Outputs run_offsets [U+1] (capacity N+1),
 * rank_runs [R] (runs per source rank: the combine send splits) and
 * *num_runs = U, all on the device.  A source rank outside [0,R) sets
 * *status (device int32, caller-zeroed) to 1.
 * Replaces the unsort, weighting and _aggregate_weighted_outputs of
 * rank_dedup_combine (veomni/distributed/moe/hiermoe/all_to_all.py:2553-2558,
 * 2266-2294). */
int pmx_ep_combine_aggregate(const void* Y, const int32_t* pos, const void* w, const int32_t* src_rank,
                             const int32_t* src_token, int64_t N, int64_t H, int32_t R, void* out,
                             int32_t* run_offsets, int32_t* rank_runs, int32_t* num_runs,
                             int32_t* status, void* workspace, size_t workspace_bytes,
                             pmx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* fp16 tensors                                                              */
/* ------------------------------------------------------------------------ */
/* The reference's fused MoE op takes bf16 or fp16 hidden states and router
 * weights (veomni/ops/kernels/moe/__init__.py:44-49) and computes in the
 * input dtype: fp32 accumulation, every rounding point in that dtype.  Each
 * entry point below is its namesake above for fp16 tensors: same arguments,
 * same checks and error codes, and every "bf16(...)" of its description is
 * round-to-nearest-even to fp16 (overflow gives inf).  The routing entry
 * points and the row copies (pmx_moe_scatter, pmx_moe_scatter_src,
 * pmx_ep_dispatch_payload) move 16-bit patterns and serve both types;
 * pmx_replica_exchange_pack/unpack take PMX_DTYPE_F16. */

int pmx_moe_gather_f16(const void* Y, const int32_t* pos, int64_t T, int32_t K, int64_t H, void* out,
                       pmx_stream_t stream);
int pmx_combine_fwd_f16(const void* Y, const int32_t* pos, const void* w, int64_t T, int32_t K, int64_t H,
                        void* out, pmx_stream_t stream);
int pmx_combine_bwd_f16(const void* dout, const void* Y, const int32_t* pos, const void* w, int64_t T,
                        int32_t K, int64_t H, void* dY, void* dw, pmx_stream_t stream);
int pmx_combine_bwd_top1_rows_f16(const void* dout, const void* Y, const int32_t* row_token, const void* w,
                                  int64_t T, int64_t H, void* dY, void* dw, pmx_stream_t stream);
int pmx_segment_sum_f16(const void* source, const int64_t* index, int64_t N, int64_t H, int64_t num_rows,
                        void* out, void* workspace, size_t workspace_bytes, pmx_stream_t stream);
int pmx_gemm_fc1_swiglu_fwd_f16(const void* X, const void* w_gate, const void* w_up, int64_t w_copy_stride,
                                const int32_t* offsets, int32_t G, int64_t A, int64_t H, int64_t I, void* gu,
                                void* act, pmx_stream_t stream);
int pmx_group_gemm_nt_f16(const void* A, const void* B, const int32_t* offsets, int32_t G, int64_t M,
                          int64_t N, int64_t K, void* C, pmx_stream_t stream);
int pmx_group_gemm_nt_combine_top1_f16(const void* A, const void* B, const int32_t* offsets, int32_t G,
                                       int64_t M, int64_t N, int64_t K, void* C, const int32_t* row_token,
                                       const void* row_weight, void* out, pmx_stream_t stream);
int pmx_group_gemm_nn_f16(const void* A, const void* B0, const void* B1, int64_t b_copy_stride,
                          int64_t b_split, const int32_t* offsets, int32_t G, int64_t M, int64_t N,
                          int64_t K, void* C, pmx_stream_t stream);
int pmx_group_gemm_nn_unpermute_top1_f16(const void* A, const void* B0, const void* B1,
                                         int64_t b_copy_stride, int64_t b_split, const int32_t* offsets,
                                         int32_t G, int64_t M, int64_t N, int64_t K,
                                         const int32_t* row_token, void* C, pmx_stream_t stream);
int pmx_gemm_fc2_dgrad_swiglu_bwd_f16(const void* dY, const void* w_down, const void* gu,
                                      const int32_t* offsets, int32_t G, int64_t A, int64_t H, int64_t I,
                                      void* dG1, pmx_stream_t stream);
int pmx_group_gemm_tn_f16(const void* A, const void* B, const int32_t* offsets, int32_t G, int64_t K,
                          int64_t M, int64_t N, void* C0, void* C1, int64_t c_copy_stride, int64_t c_split,
                          pmx_stream_t stream);
int pmx_weight_rows_f16(const void* act, const void* row_w, int64_t R, int64_t N, void* out,
                        pmx_stream_t stream);
int pmx_swiglu_bwd_weighted_f16(const void* d_act_w, const void* gu, const void* act, const void* row_w,
                                const int32_t* row_src, int64_t R, int64_t I, int64_t A, void* dG1, void* dw,
                                pmx_stream_t stream);
int pmx_replica_fold_f16(void* grads, const int32_t* copy_offsets, const int32_t* copy_slots,
                         const int64_t* slot_tokens, int32_t E, int32_t C, int64_t P, float* out,
                         int32_t writeback, int32_t* status, pmx_stream_t stream);
int pmx_ep_combine_aggregate_f16(const void* Y, const int32_t* pos, const void* w, const int32_t* src_rank,
                                 const int32_t* src_token, int64_t N, int64_t H, int32_t R, void* out,
                                 int32_t* run_offsets, int32_t* rank_runs, int32_t* num_runs,
                                 int32_t* status, void* workspace, size_t workspace_bytes,
                                 pmx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PLACEMOE_AMD_H */
