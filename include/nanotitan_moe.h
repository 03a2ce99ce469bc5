/*
 * nanotitan_moe.h — C ABI of the MI355X (gfx950) MoE expert path.
 *
 * One shared library, libnanotitan_moe.so, built by hipcc for gfx950. Every
 * entry point takes plain device pointers, sizes and a hipStream_t; launches
 * are stream-ordered, never synchronise the host and never allocate. Outputs
 * and the workspace are owned by the caller. Each call returns NT_OK or an
 * NT_ERR_* code; nt_strerror() turns a code into a message.
 *
 * Element types: activations/weights are NT_F32, NT_F64, NT_F16 or NT_BF16
 * (the four float types the reference dispatches over); gates are float32;
 * token ids, expert ids, offsets and cursors are int32. All matrices are
 * row-major and contiguous.
 *
 * Packed order ("canonical order"): assignment f = t*k + j (token t, slot j)
 * with expert e = topk[f] lands at
 *     p(f) = base[e] + #{ f' < f : topk[f'] == e }
 * i.e. a stable counting sort of the flat assignment index by expert. The
 * reference's atomic-cursor kernel leaves the order inside an expert segment
 * unspecified; its torch backend produces exactly this order
 * (src/model/torch_backend.py:58-66).
 *
 * Reference interfaces replaced (paths relative to the nanoTitan tree):
 *   csrc/bindings.cpp:9,63      count_expert_kernel       -> nt_count_experts
 *   csrc/bindings.cpp:17-22,64  pack_tokens_kernel        -> nt_pack_tokens
 *   csrc/bindings.cpp:10-16,66  combine_tokens_kernel     -> nt_combine_tokens
 *   csrc/bindings.cpp:24-30,67  combine_kernel_backward   -> nt_combine_backward
 *   csrc/bindings.cpp:32-38,80  pack_kernel_backward      -> nt_pack_backward
 *   csrc/bindings.cpp:43-47,82  grouped_gemm_kernel       -> nt_grouped_gemm
 *   csrc/bindings.cpp:53-57,88  bwd_grouped_gemm_dX_kernel-> nt_grouped_gemm_dx
 *   csrc/bindings.cpp:48-52,84  bwd_grouped_gemm_dW_kernel-> nt_grouped_gemm_dw
 * plus the torch glue of src/model/cuda_backend.py:30-37 (softmax, top-k,
 * renorm) as nt_route_topk, the glue of :46-67 (count, cumsum, pack) fused
 * into nt_dispatch, and inverse-map variants of combine and pack backward
 * used by the MoE layer.
 */
#ifndef NANOTITAN_MOE_H
#define NANOTITAN_MOE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes. */
enum nt_dtype { NT_F32 = 0, NT_F64 = 1, NT_F16 = 2, NT_BF16 = 3 };

/* Return codes. */
enum nt_status {
  NT_OK = 0,
  NT_ERR_INVALID_ARG = 1,   /* null pointer where one is required, negative size */
  NT_ERR_DTYPE = 2,         /* unknown dtype code */
  NT_ERR_TOO_MANY_EXPERTS = 3, /* E above NT_MAX_EXPERTS */
  NT_ERR_WORKSPACE = 4,     /* workspace missing or smaller than *_workspace_bytes() */
  NT_ERR_LAUNCH = 5,        /* a kernel launch failed (hipGetLastError) */
  NT_ERR_TOO_LARGE = 6,     /* a size exceeds what the kernels index (e.g. > 2^31-1 rows) */
  NT_ERR_SCRATCH = 7        /* a no-allocation call needs more than its fixed scratch */
};

#define NT_MAX_EXPERTS 1024

/* Message for a status code (static storage). */
const char* nt_strerror(int code);

/* Library version, major*10000 + minor*100 + patch. */
int nt_version(void);

/* dst[0..bytes) = src[0..bytes) with 16-byte vector loads (non-temporal) and
 * stores, four in flight per lane, on `blocks` workgroups of 256 lanes
 * (0: 8192). The
 * achievable-bandwidth reference the HBM-bound kernels are measured against:
 * a copy moves 2 * bytes. Replaces the reference's copy_kernel_vector
 * (csrc/kernels/copy_kernel.cu:25-36, benchmarks/mem_copy_benchmark.py:52-95). */
int nt_stream_copy(void* dst, const void* src, size_t bytes, int32_t blocks, hipStream_t stream);

/* Write-only and read-only ceilings beside the copy: dst[0..bytes) = value
 * (as 32-bit words), and a read of src[0..bytes) that writes nothing
 * (`sink`, one word, is written only if the XOR of the data happens to equal
 * a fixed constant). bytes and the pointers 16-byte aligned. Measurement
 * references for kernels whose traffic is mostly writes or mostly reads; no
 * counterpart in the reference. */
int nt_stream_fill(void* dst, size_t bytes, uint32_t value, hipStream_t stream);
int nt_stream_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t stream);

/* ------------------------------------------------------------------ dispatch */

/* Workspace for nt_count_experts / nt_pack_tokens / nt_dispatch with these
 * sizes (per-block expert histograms and bases). */
size_t nt_dispatch_workspace_bytes(int64_t T, int32_t k, int32_t E, int64_t d, int dtype);

/* counts[e] = #{ (t,j) : mask[t] != 0 and topk[t*k+j] == e }.
 * topk [T,k] int32, mask [T] int32 or NULL (all tokens count), counts [E].
 * Ids outside [0,E) are ignored.
 * Replaces count_expert_kernel (reference csrc/kernels/count_experts.cu:32-57). */
int nt_count_experts(const int32_t* topk, const int32_t* mask, int64_t T, int32_t k,
                     int32_t E, int32_t* counts, void* ws, size_t ws_bytes,
                     hipStream_t stream);

/* Pack token rows into expert-major order.
 * Inputs:  X [T,d] (dtype), w [T,k] f32, topk [T,k] i32,
 *          cursor [E+1] i32: cursor[e] is the first packed slot of expert e.
 * Outputs: packed_X [A_cap,d], token_id [A_cap], expert [A_cap],
 *          packed_w [A_cap] (A_cap = T*k), and inv [T*k] (may be NULL):
 *          inv[f] = packed slot of assignment f, or -1 if it was dropped.
 * Slot of assignment f: cursor[e] + #{ f' < f : topk[f'] == e } (canonical
 * order). On return cursor[e] += count[e] for e < E, the post-state the
 * reference's atomic cursor leaves. Assignments with ids outside [0,E) or a
 * slot outside [0,A_cap) are dropped (their rows are not written).
 * Replaces pack_tokens_kernel (reference csrc/kernels/pack_tokens.cu:51-111). */
int nt_pack_tokens(int dtype, const void* X, const float* w, const int32_t* topk,
                   int64_t T, int32_t k, int64_t d, int32_t E, int32_t* cursor,
                   void* packed_X, int32_t* token_id, int32_t* expert, float* packed_w,
                   int32_t* inv, void* ws, size_t ws_bytes, hipStream_t stream);

/* Fused count + exclusive scan + pack (the glue of reference
 * src/model/cuda_backend.py:46-67 plus pack_tokens_kernel):
 * counts [E], offsets [E+1] (offsets[0] = 0, offsets[e+1] = offsets[e] +
 * counts[e]), then the canonical pack with base = offsets. Outputs as in
 * nt_pack_tokens; inv may be NULL. */
int nt_dispatch(int dtype, const void* X, const float* w, const int32_t* topk, int64_t T,
                int32_t k, int64_t d, int32_t E, int32_t* counts, int32_t* offsets,
                void* packed_X, int32_t* token_id, int32_t* expert, float* packed_w,
                int32_t* inv, void* ws, size_t ws_bytes, hipStream_t stream);

/* Tokens per block of the dispatch's counting / packing for these sizes
 * (the TB of nt_route_topk_count); 0 for invalid sizes. */
int32_t nt_dispatch_block_tokens(int64_t T, int32_t k, int64_t d, int dtype);

/* nt_dispatch whose workspace already starts with the per-block counts of
 * nt_route_topk_count (TB = nt_dispatch_block_tokens(T, k, d, dtype)): the
 * same outputs, without the counting pass. The counts are only read, so a
 * second call on the same workspace gives the same outputs; the rest of the
 * workspace (up to nt_dispatch_workspace_bytes) is scratch the call
 * overwrites (the counts' scan over blocks, when E times the block count
 * is above 8192). */
int nt_dispatch_counted(int dtype, const void* X, const float* w, const int32_t* topk, int64_t T,
                        int32_t k, int64_t d, int32_t E, int32_t* counts, int32_t* offsets,
                        void* packed_X, int32_t* token_id, int32_t* expert, float* packed_w,
                        int32_t* inv, void* ws, size_t ws_bytes, hipStream_t stream);

/* Bytes of device scratch the library owns for nt_dispatch_noalloc, per GPU. */
#define NT_NOALLOC_SCRATCH_BYTES (4 << 20)

/* nt_dispatch without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the reference: its dispatch
 * allocates through torch. The workspace lives in a fixed device array of
 * NT_NOALLOC_SCRATCH_BYTES that the library owns on each GPU it runs on
 * (held until the process ends); sizes whose nt_dispatch_workspace_bytes
 * exceed it return NT_ERR_SCRATCH before any launch (two int32 tables of E
 * x ceil(T/TB) entries plus E bases: 65536 tokens x 128 experts take 2 MiB
 * at 4 KiB rows). Calls on one GPU
 * share that array and leave its contents behind (nothing in it needs to
 * start at zero); two calls that overlap on one GPU (different streams,
 * not ordered) race on it. Same outputs as nt_dispatch, bit for bit, and no
 * hipMalloc, hipFree or allocating library call. */
int nt_dispatch_noalloc(int dtype, const void* X, const float* w, const int32_t* topk, int64_t T,
                        int32_t k, int64_t d, int32_t E, int32_t* counts, int32_t* offsets,
                        void* packed_X, int32_t* token_id, int32_t* expert, float* packed_w,
                        int32_t* inv, hipStream_t stream);

/* ------------------------------------------------------------------- combine */

/* Workspace for the token-id (CSR) forms of combine and pack backward. */
size_t nt_combine_workspace_bytes(int64_t A, int64_t T);

/* out[t,:] = sum over packed rows p with token_id[p] == t, in ascending p, of
 * fl32(w[p] * float(y[p,:])), accumulated in float32 without fused
 * multiply-add. y [A,d] (dtype), token_id [A], w [A] f32, out [T,d] f32.
 * Tokens with no rows get 0. Ids outside [0,T) are ignored.
 * Replaces combine_tokens_kernel (reference csrc/kernels/combine_kernels.cu:36-78). */
int nt_combine_tokens(int dtype, const void* y, const int32_t* token_id, const float* w,
                      int64_t A, int64_t T, int64_t d, float* out, void* ws,
                      size_t ws_bytes, hipStream_t stream);

/* Same sum driven by the inverse map of nt_pack_tokens: the rows of token t
 * are inv[t*k .. t*k+k-1] (entries < 0 skipped), taken in ascending p, so
 * the result is bit-identical to nt_combine_tokens on the same pack.
 * out_dtype selects the output element type (NT_F32 for the reference
 * surface; the activation dtype folds the layer's cast into the kernel). */
int nt_combine_inv(int dtype, const void* y, const int32_t* inv, const float* w, int64_t T,
                   int32_t k, int64_t d, int out_dtype, void* out, hipStream_t stream);

/* dy[p,:] = cast(dY[t,:] * w[p]) and dw[p] = sum_h dY[t,h] * float(y[p,h])
 * with t = token_id[p]; dY [T,d] f32, dy [A,d] (dtype), dw [A] f32.
 * Rows with an id outside [0,T) get dy = 0, dw = 0.
 * Replaces combine_kernel_backward (reference csrc/kernels/backward_combine_kernel.cu:42-93). */
int nt_combine_backward(int dtype, const void* y, const int32_t* token_id, const float* w,
                        const float* dY, int64_t A, int64_t T, int64_t d, void* dy,
                        float* dw, hipStream_t stream);

/* Combine backward driven by the inverse map: one pass per token reads its
 * dY row once. dY_dtype is NT_F32 or the activation dtype. */
int nt_combine_backward_inv(int dtype, const void* y, const int32_t* inv, const float* w,
                            int dY_dtype, const void* dY, int64_t T, int32_t k, int64_t d,
                            void* dy, float* dw, hipStream_t stream);

/* dX[t,:] = cast(sum over p with token_id[p] == t, ascending p, of float(dpX[p,:]));
 * dw[t,j] = sum of dpw[p] over those p whose expert[p] first matches topk[t,j]
 * (j = the lowest slot with topk[t,j] == expert[p]; rows with no match add
 * nothing). dpX [A,d], dpw [A] f32, token_id/expert [A], topk [T,k],
 * dX [T,d] (dtype), dw [T,k] f32.
 * Replaces pack_kernel_backward (reference csrc/kernels/backward_pack_kernel.cu:46-101). */
int nt_pack_backward(int dtype, const void* dpX, const float* dpw, const int32_t* token_id,
                     const int32_t* expert, const int32_t* topk, int64_t A, int64_t T,
                     int32_t k, int64_t d, void* dX, float* dw, void* ws, size_t ws_bytes,
                     hipStream_t stream);

/* Pack backward driven by the inverse map: dX[t,:] = cast(sum of dpX rows
 * inv[t*k+j] in ascending slot order), dw[t,j] = dpw[inv[t*k+j]] (0 when
 * inv < 0). */
int nt_pack_backward_inv(int dtype, const void* dpX, const float* dpw, const int32_t* inv,
                         int64_t T, int32_t k, int64_t d, void* dX, float* dw,
                         hipStream_t stream);

/* nt_pack_backward_inv followed by nt_route_topk_backward on its dw, in one
 * launch when k <= 8: dX as nt_pack_backward_inv, and dlogits [T,E] f32 the
 * router gradient for gates [T,k], topk [T,k] and dgates dw (bit-identical
 * to the two calls). dw [T,k] is optional (NULL: not written) when k <= 8
 * and required above (the two launches then run). The router's limits hold
 * (k <= E, k <= 32, E <= NT_MAX_EXPERTS) and are checked before any launch.
 * Replaces the pack
 * backward (reference csrc/kernels/backward_pack_kernel.cu:10-44) and the
 * backward of the router's softmax / top-k / renormalisation, which the
 * reference leaves to torch autograd (src/model/cuda_backend.py:30-37),
 * for a layer whose gates feed only the dispatch. */
int nt_pack_backward_inv_route(int dtype, const void* dpX, const float* dpw, const int32_t* inv,
                               const float* gates, const int32_t* topk, int64_t T, int32_t k,
                               int64_t d, int32_t E, void* dX, float* dlogits, float* dw,
                               hipStream_t stream);

/* -------------------------------------------------------------------- router */

/* Router gate for logits [T,E] f32: top-k experts by logit (ties to the
 * lower expert id; equal to the top-k of softmax(logits)), gates [T,k] f32 =
 * the softmax of the k selected logits (= the selected probabilities
 * renormalised to sum 1), topk [T,k] i32 in descending order, and optionally
 * probs [T,E] = softmax(logits) (NULL to skip). k <= 32.
 * Replaces the torch glue of reference src/model/cuda_backend.py:30-37. */
int nt_route_topk(const float* logits, int64_t T, int32_t E, int32_t k, float* gates,
                  int32_t* topk, float* probs, hipStream_t stream);

/* nt_route_topk with the expert count fused in: the same gates / topk /
 * probs, plus hist[e*nb + b] = #{(t, j) : b*TB <= t < (b+1)*TB, topk[t,j] = e}
 * for every block b < nb = ceil(T/TB), each entry written (no zero-fill
 * needed). With TB = nt_dispatch_block_tokens(T, k, d, dtype) and hist at
 * the start of the dispatch workspace, nt_dispatch_counted skips its own
 * counting pass. E <= NT_MAX_EXPERTS. Replaces the router glue and
 * count_expert_kernel (reference src/model/cuda_backend.py:30-52,
 * csrc/kernels/count_experts.cu:8-57). */
int nt_route_topk_count(const float* logits, int64_t T, int32_t E, int32_t k, float* gates,
                        int32_t* topk, float* probs, int32_t TB, int32_t* hist,
                        hipStream_t stream);

/* Gradient of nt_route_topk's gates: dlogits [T,E] f32, zero except at the
 * selected experts, where dlogits = gate * (dgate - sum_j dgate_j * gate_j). */
int nt_route_topk_backward(const float* gates, const int32_t* topk, const float* dgates,
                           int64_t T, int32_t E, int32_t k, float* dlogits, hipStream_t stream);

/* ------------------------------------------------------------- grouped GEMM */

/* Workspace for nt_grouped_gemm_dw and the paired dW + dX calls with these
 * sizes (the forward and dX GEMMs need none; pass NULL, 0). It holds 256
 * bytes of tile counters (paired calls), then the fp32 partial sums of
 * experts whose reduction is split (skewed routing): at most 256 MiB plus
 * one K*N*4 slab, and 8 bytes per slab and 256x256 dW tile of arrival
 * counters (a paired call sums the partial sums in its own launch); 256
 * bytes when no split can occur. A smaller or NULL
 * workspace is accepted: dW then runs unsplit (and unpaired). Its contents
 * need no initialisation: the counters carry a per-launch tag, and every
 * slab a launch reads it has written. A paired call made while its stream
 * is being captured into a HIP graph clears its counters with a kernel
 * launched just before it, so every replay of the graph starts them from
 * zero. Calls that overlap in time must not share a workspace. */
size_t nt_grouped_gemm_workspace_bytes(int dtype, int32_t E, int64_t A, int64_t K, int64_t N);

/* out[a,:] = X[a,:] @ W[e] for a in [offsets[e], offsets[e+1]), float32
 * accumulation, cast to dtype. X [A,K], W [E,K,N], out [A,N], offsets [E+1]
 * non-decreasing with offsets[E] <= A. Rows >= offsets[E] are not written.
 * Replaces grouped_gemm_kernel (reference csrc/kernels/grouped_gemm.cu:43-91). */
int nt_grouped_gemm(int dtype, const void* X, const int32_t* offsets, const void* W, int32_t E,
                    int64_t A, int64_t K, int64_t N, void* out, void* ws, size_t ws_bytes,
                    hipStream_t stream);

/* dX[a,:] = dOut[a,:] @ W[e]^T. W [E,K,N], dOut [A,N], dX [A,K].
 * Replaces bwd_grouped_gemm_dX_kernel (reference csrc/kernels/bwd_grouped_gemm_dX.cu:46-96). */
int nt_grouped_gemm_dx(int dtype, const void* W, const int32_t* offsets, const void* dOut,
                       int32_t E, int64_t A, int64_t K, int64_t N, void* dX, void* ws,
                       size_t ws_bytes, hipStream_t stream);

/* Up-projection with the GELU (erf form) fused into the epilogue. With
 * h = X_e @ W[e] rounded to dtype (as nt_grouped_gemm writes it), stores
 * act = gelu(h) and act_grad = gelu'(h), both [A,N] and rounded once; h
 * itself is not stored (the backward needs only act_grad). The reference
 * runs grouped_gemm_kernel and then the activation
 * (src/model/feed_fwd.py:107-112, with the configs' GELU in place of SiLU);
 * no single reference entry point corresponds. */
int nt_grouped_gemm_gelu(int dtype, const void* X, const int32_t* offsets, const void* W,
                         int32_t E, int64_t A, int64_t K, int64_t N, void* act, void* act_grad,
                         void* ws, size_t ws_bytes, hipStream_t stream);

/* dX GEMM with the GELU backward fused into the epilogue:
 * dH = (dOut @ W[e]^T, rounded) * act_grad, rounded once, with act_grad the
 * gelu'(h) nt_grouped_gemm_gelu stored. W [E,K,N], dOut [A,N], act_grad and
 * dH [A,K]. Replaces bwd_grouped_gemm_dX_kernel followed by the
 * activation's backward (reference csrc/kernels/bwd_grouped_gemm_dX.cu:46-96,
 * then autograd). */
int nt_grouped_gemm_dx_gelu(int dtype, const void* W, const int32_t* offsets, const void* dOut,
                            const void* act_grad, int32_t E, int64_t A, int64_t K, int64_t N,
                            void* dH, void* ws, size_t ws_bytes, hipStream_t stream);

/* SwiGLU up-projection: the gate and value GEMMs of each output tile run
 * in one kernel (the B tiles of W_gate and W_val side by side) and the
 * epilogue writes gate = X_e @ W_gate[e], value = X_e @ W_val[e] (each
 * rounded to dtype) and hidden = silu(gate) * value (silu rounded, then the
 * product rounded), all [A,N]; gate and value are what the backward needs.
 * W_gate, W_val [E,K,N]. Replaces the two grouped_gemm_kernel calls and the
 * activation of the reference's SwiGLU ExpertFFN
 * (src/model/feed_fwd.py:107-110). */
int nt_grouped_gemm_swiglu(int dtype, const void* X, const int32_t* offsets, const void* W_gate,
                           const void* W_val, int32_t E, int64_t A, int64_t K, int64_t N,
                           void* hidden, void* gate, void* value, void* ws, size_t ws_bytes,
                           hipStream_t stream);

/* dX GEMM with the SwiGLU backward in its epilogue: with
 * dhidden = dOut @ W[e]^T rounded to dtype, writes
 * dvalue = dhidden * silu(gate) and dgate = (dhidden * value) * silu'(gate)
 * (each product rounded where torch's autograd of silu(gate) * value
 * rounds it). W [E,K,N] (W_out), dOut [A,N], gate / value / dgate / dvalue
 * [A,K]. Replaces bwd_grouped_gemm_dX_kernel followed by the autograd of
 * the activation (reference csrc/kernels/bwd_grouped_gemm_dX.cu:46-96,
 * src/model/feed_fwd.py:110). */
int nt_grouped_gemm_dx_swiglu(int dtype, const void* W, const int32_t* offsets, const void* dOut,
                              const void* gate, const void* value, int32_t E, int64_t A,
                              int64_t K, int64_t N, void* dgate, void* dvalue, void* ws,
                              size_t ws_bytes, hipStream_t stream);

/* Two dX products summed in one GEMM over the concatenated reduction:
 * dX[a,:] = dOut1[a,:] @ W1[e]^T + dOut2[a,:] @ W2[e]^T, fp32 accumulation,
 * one rounding. W1, W2 [E,K,N], dOut1, dOut2 [A,N], dX [A,K]. Replaces the
 * two bwd_grouped_gemm_dX_kernel calls of the SwiGLU gate and value
 * projections and the autograd sum of their results
 * (reference csrc/kernels/bwd_grouped_gemm_dX.cu:46-96, src/model/feed_fwd.py:108-109). */
int nt_grouped_gemm_dx2(int dtype, const void* W1, const void* W2, const int32_t* offsets,
                        const void* dOut1, const void* dOut2, int32_t E, int64_t A, int64_t K,
                        int64_t N, void* dX, void* ws, size_t ws_bytes, hipStream_t stream);

/* dW[e] = X_e^T @ dOut_e summed over the rows of expert e (zero for an empty
 * expert). X [A,K], dOut [A,N], dW [E,K,N]. An expert with more rows than
 * about 1.25 times a workgroup's share of the reduction (skewed routing) is
 * reduced in chunks of about half a share, whose fp32 partials go to ws
 * and are summed in chunk order, so no single tile outlasts the rest: by a
 * second kernel here, inside the launch in the paired dW + dX calls (the
 * last chunk of a tile to arrive sums them). Deterministic: the chunks
 * depend only on the sizes (the share is planned for 256 CUs on every
 * device) and every tile is summed in chunk order; the paired calls'
 * atomic counters only decide which workgroup does the sum, never its
 * order.
 * Replaces bwd_grouped_gemm_dW_kernel (reference csrc/kernels/bwd_grouped_gemm_dW.cu:43-86). */
int nt_grouped_gemm_dw(int dtype, const void* X, const int32_t* offsets, const void* dOut,
                       int32_t E, int64_t A, int64_t K, int64_t N, void* dW, void* ws,
                       size_t ws_bytes, hipStream_t stream);

/* nt_grouped_gemm_dw (dW = X^T dOut, [E,K,N]) and nt_grouped_gemm_dx
 * (dX = dOut W^T, [A,K]) in one call, for the backward of one expert
 * projection: the two read the same dOut and are otherwise independent.
 * When the dW has too few 256x256 tiles to fill the device and there are at
 * most 16 experts, one kernel launch runs both side by side (the dW on
 * 256x256 tiles, one per workgroup, the dX on the remaining CUs and then on
 * the dW's as they finish); otherwise they run one after the other. Outputs are bit-identical to the two separate calls. ws: the dW
 * workspace (nt_grouped_gemm_workspace_bytes). Replaces the pair of calls in
 * GroupedGEMM_FN.backward (reference
 * src/model/moe_ops.py:117-125; csrc/kernels/bwd_grouped_gemm_dW.cu:43-86,
 * bwd_grouped_gemm_dX.cu:46-96). */
int nt_grouped_gemm_dw_dx(int dtype, const void* X, const void* W, const int32_t* offsets,
                          const void* dOut, int32_t E, int64_t A, int64_t K, int64_t N, void* dW,
                          void* dX, void* ws, size_t ws_bytes, hipStream_t stream);

/* The same pairing for the GELU FFN's down projection: dW = act^T dOut
 * (nt_grouped_gemm_dw) and dH = (dOut W^T) * act_grad
 * (nt_grouped_gemm_dx_gelu). act, act_grad [A,K]; W [E,K,N]; dOut [A,N]. */
int nt_grouped_gemm_dw_dx_gelu(int dtype, const void* act, const void* W, const int32_t* offsets,
                               const void* dOut, const void* act_grad, int32_t E, int64_t A,
                               int64_t K, int64_t N, void* dW, void* dH, void* ws,
                               size_t ws_bytes, hipStream_t stream);

/* The same pairing for the SwiGLU FFN's output projection: dW = hidden^T
 * dOut (nt_grouped_gemm_dw) and (dgate, dvalue) from dhidden = dOut W^T
 * (nt_grouped_gemm_dx_swiglu). hidden, gate, value, dgate, dvalue [A,K]. */
int nt_grouped_gemm_dw_dx_swiglu(int dtype, const void* hidden, const void* W,
                                 const int32_t* offsets, const void* dOut, const void* gate,
                                 const void* value, int32_t E, int64_t A, int64_t K, int64_t N,
                                 void* dW, void* dgate, void* dvalue, void* ws, size_t ws_bytes,
                                 hipStream_t stream);

/* And for its input projections: dW1 = X^T dOut1 (nt_grouped_gemm_dw, the
 * gate weights' gradient) and dX = dOut1 W1^T + dOut2 W2^T
 * (nt_grouped_gemm_dx2). X, dX [A,K]; W1, W2 [E,K,N]; dOut1, dOut2 [A,N]. */
int nt_grouped_gemm_dw_dx2(int dtype, const void* X, const void* W1, const void* W2,
                           const int32_t* offsets, const void* dOut1, const void* dOut2,
                           int32_t E, int64_t A, int64_t K, int64_t N, void* dW1, void* dX,
                           void* ws, size_t ws_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOTITAN_MOE_H */
