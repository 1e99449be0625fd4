/*
 * i4moe.h -- C ABI of the MI355X (gfx950) int4 clock-path library.
 *
 * One shared library (libi4moe.so) replaces the quantized compute that runs
 * Qwen3-Omni Thinker layers 0-23 in thecodacus/qwen3-omni-duplex:
 *
 *   - the int4 dequant-GEMV   (src/duplex/streaming/triton_dequant_gemv.py:32-113)
 *   - the packed Linear       (src/duplex/streaming/triton_dequant_gemv.py:125-159)
 *   - the fused int4 MoE block (src/duplex/streaming/fused_packed_moe.py:83-275)
 *
 * Conventions shared by every entry point:
 *   - all functions are extern "C" and return int: 0 = I4_OK, < 0 = error code
 *     (i4_strerror() turns it into a static string);
 *   - the library never allocates, frees or synchronises: outputs and
 *     workspaces are caller memory, work is only enqueued on `stream`
 *     (so every call can be captured into a hipGraph);
 *   - every pointer is a device pointer unless stated otherwise and must be
 *     16-byte aligned when it points to packed weights or activations;
 *   - shapes are validated on the host before anything is launched; an
 *     invalid call launches nothing;
 *   - an expert id outside [0, E) is never dereferenced: the affected output
 *     rows are written as NaN (the reference faults with an illegal address,
 *     src/duplex/streaming/fused_packed_moe.py:227-229).
 *
 * Weight formats (W is the logical [N out][K in] matrix of y = W x):
 *   I4_LAYOUT_CT  -- compressed-tensors "pack-quantized", the reference's own
 *                    format (src/duplex/quant/dequant.py:23-27,
 *                    src/duplex/streaming/fused_packed_moe.py:7-11,54-65):
 *                      packed [E][N][K/8] int32, column k = 8m+i of a row is
 *                             nibble i (bits 4i..4i+3) of word m;
 *                      scale  [E][N][NG],  NG = ceil(K/group);
 *                      zeros  NULL (symmetric, zero point 8, the reference) or
 *                             [E][N][ceil(NG/8)] int32, group g in nibble g%8
 *                             of word g/8.
 *                    value = (nibble - zero) * scale.
 *   I4_LAYOUT_AWQ -- AutoAWQ GEMM packing:
 *                      qweight [E][K][N/8] int32, nibble slot i of word w holds
 *                             column 8w + {0,2,4,6,1,3,5,7}[i];
 *                      qzeros  [E][NG][N/8] int32, same packing;
 *                      scales  [E][NG][N].
 *   I4_LAYOUT_TILE -- this library's load-time layout for the MoE kernels (no
 *                    reference counterpart; built by i4_repack_tile).  The CT
 *                    words regrouped so that one 16-byte load of lane (row r,
 *                    k-group j) holds word j of the four 32-column chunks of a
 *                    128-column superchunk, and one wavefront load is 1 KB of
 *                    contiguous memory (16 rows x 4 k-groups):
 *                      packed [E][N/16][K/128][16][4][4] int32, element
 *                             [e][b][s][r][j][t] = CT word 4 (4s + t) + j of
 *                             row 16b + r with its nibbles interleaved: slot
 *                             i holds column 8m + {0,2,4,6,1,3,5,7}[i] (the
 *                             AWQ order), so nibbles i and i + 4 are two
 *                             adjacent columns;
 *                      scale  [E][N/16][NG][16], element [e][b][g][r] = CT
 *                             scale of row 16b + r, group g;
 *                      zeros  NULL or [E][N/16][ceil(NG/8)][16] int32, the CT
 *                             zero words of row 16b + r.
 *                    Needs N % 16 == 0 and K % 128 == 0.
 */
#ifndef I4MOE_H
#define I4MOE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define I4_ABI_VERSION 9

/* status codes */
#define I4_OK               0
#define I4_ERR_NULL        -1  /* a required pointer is NULL                     */
#define I4_ERR_SHAPE       -2  /* dimension out of range or inconsistent         */
#define I4_ERR_DTYPE       -3  /* unsupported element type                       */
#define I4_ERR_ALIGN       -4  /* pointer not 16-byte aligned                    */
#define I4_ERR_LAYOUT      -5  /* unsupported packed layout for this entry point */
#define I4_ERR_GROUP       -6  /* group size not a multiple of 32                */
#define I4_ERR_WORKSPACE   -7  /* workspace missing or too small                 */
#define I4_ERR_LAUNCH      -8  /* the HIP runtime rejected a kernel launch       */
#define I4_ERR_STRIDE      -9  /* expert or row stride smaller than its data     */
#define I4_ERR_HANDOFF    -10  /* a decode wait for activations gave up (NaN out) */
#define I4_ERR_SCRATCH    -11  /* call needs more than the static scratch holds   */

/* element types */
#define I4_F32  0
#define I4_F16  1
#define I4_BF16 2

/* packed layouts */
#define I4_LAYOUT_CT   0
#define I4_LAYOUT_AWQ  1
#define I4_LAYOUT_TILE 2

/* One stacked int4 weight: E experts of a [N][K] matrix.  E = 1 is a plain
 * Linear.  *_estride are element strides between experts; 0 means densely
 * stacked.  Mirrors the (packed, scale) pair that
 * src/duplex/streaming/fused_packed_moe.py:68-80 (_stack_packed) builds, plus
 * the optional zero points of the AWQ format. */
typedef struct i4_qweight {
  const int32_t* packed;
  const void*    scale;
  const int32_t* zeros;
  int64_t        packed_estride;
  int64_t        scale_estride;
  int64_t        zeros_estride;
  int32_t        layout;       /* I4_LAYOUT_*                        */
  int32_t        group;        /* quantisation group along K, %32==0 */
  int32_t        scale_dtype;  /* I4_F32 / I4_F16 / I4_BF16          */
  int32_t        E, N, K;
} i4_qweight;

/* One Thinker MoE block, as FusedPackedMoE stores it
 * (src/duplex/streaming/fused_packed_moe.py:112,117-122,166-169).
 * gate_up / down are in I4_LAYOUT_CT (the decode kernels read whole rows) or
 * I4_LAYOUT_TILE; gate_up_tile / down_tile are optional tile copies of the
 * same weights (packed == NULL: absent) for the T > 1 MFMA kernels, which read
 * tiles only.  T = 1 uses gate_up / down; T > 1 uses the tile copies, or
 * gate_up / down when those are tiles (else I4_ERR_LAYOUT). */
typedef struct i4_moe_weights {
  i4_qweight  gate_up;    /* [E][2I][H]: rows [0,I) gate_proj, [I,2I) up_proj */
  i4_qweight  down;       /* [E][H][I]                                       */
  const void* router_w;   /* [E][H] dense, in the activation dtype; may be
                             NULL when logits are passed to i4_moe_forward    */
  const void* norm_w;     /* [H] in the activation dtype, or NULL.  When set,
                             the block runs on RMSNorm(x) -- the decoder
                             layer's post_attention_layernorm in front of the
                             MoE (transformers Qwen3OmniMoeThinkerTextRMSNorm:
                             w * (x * rsqrt(mean(x^2) + eps)).to(dtype)) --
                             while the residual stays the un-normalised input.
                             Requires router_w.                               */
  float       norm_eps;
  i4_qweight  gate_up_tile;
  i4_qweight  down_tile;
} i4_moe_weights;

int         i4_abi_version(void);
const char* i4_strerror(int code);

/* dequant_gemv (src/duplex/streaming/triton_dequant_gemv.py:85-113):
 *   out[j][n] = sum_k W[sel[j]][n][k] * x[j * x_stride + k],  j < k_sel
 * x_stride = 0 shares one activation row across the selected experts (the
 * gate_up call, fused_packed_moe.py:255); x_stride = K gives each expert its
 * own row (the down call, fused_packed_moe.py:261).  Accumulation is fp32.
 * out is [k_sel][N] in out_dtype (I4_F32 matches the reference).  Either
 * layout runs in one launch.  CT and most AWQ shapes need no workspace
 * (i4_dq_gemv_workspace_bytes() returns 0; NULL / 0 is accepted).  An AWQ
 * weight with N % 32 == 0 whose K-complete launch would stream more than 2048
 * rows per CU (K x ceil(N / 8 * k_sel / 256) > 2048, e.g. 2048 -> 4096 and
 * 4096 -> 2048), with k_sel <= 8 and partials of at most 8 MiB, is split along K
 * when the caller passes the workspace that i4_dq_gemv_workspace_bytes() names
 * (256-byte aligned, one workspace per stream); with a NULL workspace it runs
 * K-complete, a smaller one is I4_ERR_WORKSPACE.  The split launch hands each
 * slice's partial sums to the last slice of its column strip inside the launch,
 * tagged with a number the library gives every call, so the workspace needs no
 * initial contents and a partial left by an earlier call is never taken.  Its
 * first int32 is a status word: a call whose hand-over wait gave up (its outputs
 * are NaN then) stores I4_ERR_HANDOFF there; calls never clear it, so zero it when
 * the workspace is allocated and read it (after the stream) to learn of a failure.
 * AWQ scales must be 16-byte aligned (also between experts).
 * A group at least as long as K is one scale per output row (the per-channel
 * branch of quant/dequant.py:75-76); a K that is not a multiple of the group
 * leaves a short last group (NG = ceil(K / group) scales per row). */
int    i4_dq_gemv(const void* x, int x_dtype, int64_t x_stride,
                  const i4_qweight* w, const int32_t* sel, int k_sel,
                  void* out, int out_dtype,
                  void* workspace, size_t workspace_bytes, hipStream_t stream);
size_t i4_dq_gemv_workspace_bytes(const i4_qweight* w, int k_sel);
/* i4_dq_gemv with a caller bound on the split launch's hand-over wait (i4_dq_gemv
 * uses 2^20 polls); reducers_only = 1 launches only the last slice of every strip,
 * whose partials then never arrive: the wait gives up after max_polls polls (NaN
 * outputs, I4_ERR_HANDOFF in the status word) and every kernel exits.  No reference
 * counterpart: the host's way of testing the bounded wait.  I4_ERR_WORKSPACE /
 * I4_ERR_LAYOUT when the call would not run split. */
int    i4_dq_gemv_bounded(const void* x, int x_dtype, int64_t x_stride,
                          const i4_qweight* w, const int32_t* sel, int k_sel,
                          void* out, int out_dtype, void* workspace, size_t workspace_bytes,
                          int max_polls, int reducers_only, hipStream_t stream);

/* TritonPackedLinear.forward (src/duplex/streaming/triton_dequant_gemv.py:151-159):
 *   y[m][n] = sum_k W[n][k] * x[m][k] (+ bias[n]),  m < M, expert 0 of w.
 * One launch for all M rows (the reference launches once per row).  bias is
 * nullable and in y_dtype.  A CT or AWQ weight runs the dequant-GEMV for
 * every row; a weight in I4_LAYOUT_TILE (E = 1, N % 128 == 0) runs the MFMA
 * tile kernel over 64-row tiles, each weight tile streamed once per 64 rows
 * (the path for prefill and other M > 1 batches); when that grid is small it
 * is split along K into fp32 partials in the workspace and summed in a fixed
 * order.  i4_linear_workspace_bytes gives the workspace (0: none needed); for
 * an AWQ weight it is i4_dq_gemv's split-K workspace (M <= 8), with its status
 * word. */
int    i4_linear(const void* x, int x_dtype, int M, const i4_qweight* w,
                 const void* bias, void* y, int y_dtype,
                 void* workspace, size_t workspace_bytes, hipStream_t stream);
size_t i4_linear_workspace_bytes(const i4_qweight* w, int M);

/* y = W RMSNorm(x) (+ bias) for every row of x in one launch: the decoder's
 * input_layernorm in front of the fused q|k|v projection (transformers
 * Qwen3OmniMoeThinkerTextDecoderLayer.forward, modeling_qwen3_omni_moe.py:1547-1549;
 * the reference runs the norm, then TritonPackedLinear, triton_dequant_gemv.py:151-159).
 * Each workgroup normalises its staged row with the arithmetic of i4_rmsnorm, so the
 * result equals i4_rmsnorm followed by i4_linear bit for bit.  CT weights, K <= 4096. */
int    i4_rmsnorm_linear(const void* x, int x_dtype, int M, const void* norm_w, float eps,
                         const i4_qweight* w, const void* bias, void* y, int y_dtype,
                         hipStream_t stream);

/* unpack4 (src/duplex/streaming/fused_packed_moe.py:54-65): raw nibbles of
 * every expert in logical [E][N][K] order as uint8 0..15 (the reference's
 * signed value is nibble - 8).  Same device decode as the GEMV kernels. */
int    i4_unpack(const i4_qweight* w, uint8_t* out, hipStream_t stream);

/* FusedPackedMoE._dequant (src/duplex/streaming/fused_packed_moe.py:183-189):
 * dense [E][N][K] = (nibble - zero) * scale, computed in fp32 and rounded
 * once to out_dtype. */
int    i4_dequant(const i4_qweight* w, void* out, int out_dtype, hipStream_t stream);

/* Load-time repack of an AWQ weight into the CT layout with explicit zeros
 * (the kernel-native format).  Writes expert e of src into rows
 * [row_offset, row_offset + src->N) of a CT destination that has dst_rows
 * rows per expert; dst_scale is in src->scale_dtype.  Used to build the
 * gate|up concatenation of fused_packed_moe.py:122 from AWQ experts. */
int    i4_repack_awq_to_ct(const i4_qweight* src, int32_t* dst_packed, void* dst_scale,
                           int32_t* dst_zeros, int dst_rows, int row_offset,
                           hipStream_t stream);

/* Load-time repack of a CT or AWQ weight into I4_LAYOUT_TILE (no reference
 * counterpart: it replaces the stacking of _stack_packed,
 * fused_packed_moe.py:68-80, for the MoE kernels).  Expert e of src goes to
 * rows [row_offset, row_offset + src->N) of a destination with dst_rows rows
 * per expert (dst_rows and row_offset multiples of 16, so gate and up can be
 * concatenated); dst_scale is in src->scale_dtype.  dst_zeros may be NULL only
 * when src has no zeros (the symmetric zero point 8 is then implied). */
int    i4_repack_tile(const i4_qweight* src, int32_t* dst_packed, void* dst_scale,
                      int32_t* dst_zeros, int dst_rows, int row_offset, hipStream_t stream);

/* Router half of FusedPackedMoE.forward (fused_packed_moe.py:195):
 *   logits[t][e] = sum_h xn[t][h] * router_w[e][h], fp32 accumulation,
 * rounded to x_dtype like the reference's half-precision gate Linear.
 * xn = x, or RMSNorm(x) with weight norm_w when norm_w is not NULL; xn_out
 * ([T][H]) receives xn.  xn_out may be NULL when T == 1 (the norm then stays
 * in registers); with norm_w and T > 1 it is required (I4_ERR_NULL). */
int    i4_router_logits(const void* x, int x_dtype, int T, int H,
                        const void* router_w, int E, const void* norm_w, float norm_eps,
                        void* xn_out, void* logits, hipStream_t stream);

/* Routing (fused_packed_moe.py:195-199): softmax in fp32 over E logits,
 * top-k, optional renormalisation.  Ties are broken by the lower expert id.
 * sel [T][topk] int32 (descending weight); w_f32 [T][topk] (nullable);
 * w_half [T][topk] in w_half_dtype (nullable; the reference's w.to(x.dtype)). */
int    i4_route_topk(const void* logits, int logits_dtype, int T, int E, int topk,
                     int renorm, int32_t* sel, float* w_f32, void* w_half,
                     int w_half_dtype, hipStream_t stream);

/* FusedPackedMoE.forward (fused_packed_moe.py:191-263), hidden states in and
 * out, optional residual: out[t] = residual[t] + sum_j w[t][j] * down(
 * silu(gate(x[t])) * up(x[t]))_{sel[t][j]}.  Routing comes from
 * weights->router_w, or from `logits` ([T][E], x_dtype) when router_w is
 * NULL.  The activation is rounded to x_dtype between the two projections as
 * in the reference (fused_packed_moe.py:257); everything else is fp32 and the
 * output is rounded once to x_dtype.  sel_out / w_out (nullable) receive the
 * routing. */
int    i4_moe_forward(const void* x, int x_dtype, int T, const i4_moe_weights* weights,
                      int topk, int renorm, const void* logits, const void* residual,
                      void* out, int32_t* sel_out, float* w_out,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);
/* Workspace of i4_moe_forward (scratch for logits, routing, expert lists and
 * intermediate activations).  One word carries over from call to call: the first
 * four bytes hold the epoch of the 2..64-token routing launch, whose router
 * workgroups hand their logits to the ranking waves as (value pair, tag) words
 * tagged with it and which a later launch of the call advances, so no word left by
 * an earlier call can pass for this call's; any starting value works (no
 * initialisation; a word left by something else passes with odds 2^-32).  Calls
 * that share one workspace must not overlap. */
size_t i4_moe_workspace_bytes(int T, int H, int I, int E, int topk);

/* i4_moe_forward for 2 <= T <= 64 tokens with the bound of its in-launch wait set by
 * the caller (no reference counterpart: the reference runs the two projections as
 * separate calls, fused_packed_moe.py:255-261).  At these sizes both expert
 * projections run as one launch whose down workgroups wait, at most max_polls polls per
 * 128-column block, for the activations that the launch's gate_up workgroups write
 * (i4_moe_forward bounds it at 2^20, which a launch dispatched in block order never
 * reaches).  down_only = 1 launches the down workgroups alone, so every wait gives up:
 * the rows they own come out NaN (so does out) and the status word at
 * i4_moe_status_offset(T, H, I, E, topk) holds I4_ERR_HANDOFF; every kernel still
 * exits.  down_only = 2 bounds the routing launch's wait instead (router logits and
 * top-k in one launch, whose ranking waves wait for their token's logits; the router
 * in the block, E <= 128, E % 4 == 0, else I4_ERR_SHAPE) and launches its ranking
 * waves alone: every routing weight, and so out, is NaN and the status word (not
 * cleared first in this mode) holds I4_ERR_HANDOFF.  For testing the bounded waits
 * from the host.  I4_ERR_SHAPE outside 2..64 tokens, for other modes, or when gate_up
 * and down use different group sizes (then nothing waits). */
int    i4_moe_forward_bounded(const void* x, int x_dtype, int T, const i4_moe_weights* weights,
                              int topk, int renorm, const void* logits, const void* residual,
                              void* out, void* workspace, size_t workspace_bytes, int max_polls,
                              int down_only, hipStream_t stream);

/* Byte offset, inside the workspace of i4_moe_forward / i4_moe_stack_forward
 * with these sizes, of an int32 status word that every call rewrites on the
 * device: I4_OK, or I4_ERR_HANDOFF when a workgroup of the single-launch decode
 * layer, or a down workgroup of the 2..64-token launch that runs both expert
 * projections, gave up waiting for the activations of its own launch (its output
 * rows are then NaN), or a ranking wave of the 2..64-token routing launch (router
 * logits and top-k in one launch, E <= 128) gave up waiting for its token's logits
 * (its routing weights, and so its output row, are then NaN).  The host reads it after the stream has finished the call; a
 * stack call reports a give-up in any of its layers.  The wait only ends that
 * way if the launch's workgroups are not dispatched in block order, which the
 * wait assumes (no reference counterpart: the reference faults instead,
 * src/duplex/streaming/fused_packed_moe.py:227-229). */
size_t i4_moe_status_offset(int T, int H, int I, int E, int topk);

/* The consumer half of the single-launch decode layer on its own: the down
 * workgroups of i4_moe_forward's T = 1 experts launch rank the [E_r] logits
 * (as fused_packed_moe.py:195-199 does), wait for act [topk][I] (x_dtype,
 * slot order of the ranking) by polling it until no value still holds the
 * pending pattern 0xFFFF, then compute out = residual + sum_j w_j
 * down_{sel_j}(act_j) (fused_packed_moe.py:261-262).  Each workgroup polls at
 * most max_polls times; one that gives up writes NaN to its output rows and
 * I4_ERR_HANDOFF to *status (int32, device; I4_OK is written first by the
 * caller or left from before: the kernel only ever stores the failure).  For
 * activations produced by another launch running concurrently, and for
 * testing the bounded wait from the host.  CT down weights, topk <= 8. */
int    i4_moe_down_wait(const void* act, int x_dtype, const i4_qweight* down,
                        const void* logits, int E_r, int topk, int renorm,
                        const void* residual, void* out, int32_t* status, int max_polls,
                        hipStream_t stream);

/* The two expert stages of one decode token with routing already known --
 * the body of the reference's per-token loop (fused_packed_moe.py:231-263):
 *   i4_moe_gate_up:      act[j][:] = silu(gate_e(x)) * up_e(x), e = sel[j],
 *                        rounded to x_dtype (fused_packed_moe.py:255-257);
 *   i4_moe_down_combine: out = residual + sum_j w[j] * down_{sel[j]}(act[j])
 *                        (fused_packed_moe.py:261-262), fixed j order.
 * x, residual and out are [H]; act is [topk][I]; sel [topk]; w [topk] fp32.
 * The weights are in I4_LAYOUT_CT or I4_LAYOUT_TILE. */
int    i4_moe_gate_up(const void* x, int x_dtype, const i4_qweight* gate_up,
                      const int32_t* sel, int topk, void* act, hipStream_t stream);
/* Routing (fused_packed_moe.py:195-199) and the gate_up stage of one decode
 * token in one launch: every workgroup ranks the E_r half-precision logits
 * itself; sel_out / w_out ([topk], fp32) receive the routing for the down
 * stage.  This is the decode path i4_moe_forward takes at T = 1. */
int    i4_moe_route_gate_up(const void* x, int x_dtype, const i4_qweight* gate_up,
                            const void* logits, int E_r, int topk, int renorm,
                            int32_t* sel_out, float* w_out, void* act, hipStream_t stream);
int    i4_moe_down_combine(const void* act, int x_dtype, const i4_qweight* down,
                           const int32_t* sel, const float* w, int topk,
                           const void* residual, void* out, hipStream_t stream);

/* The Thinker[0:24] MoE stack of src/duplex/streaming/clock.py:168-171 with
 * only the MoE blocks and residual adds kept: h <- h + moe_l(h) for
 * l < n_layers.  x and out are [T][H]; x is not modified.  At T = 1 with top-8
 * blocks of CT experts and H = 1024 or 2048 every layer runs the XCD-local
 * pair of launches below (i4_moe_route_sum, i4_moe_experts_x; i4_moe_sum after
 * the last layer), otherwise i4_moe_forward per layer; both give the same
 * result bit for bit. */
int    i4_moe_stack_forward(const void* x, int x_dtype, int T,
                            const i4_moe_weights* layers, int n_layers, int topk,
                            int renorm, void* out, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);
size_t i4_moe_stack_workspace_bytes(int T, int H, int I, int E, int topk);

/* The launches of one decode layer (T = 1) of i4_moe_stack_forward on an MI355X,
 * the pieces of FusedPackedMoE.forward's Triton branch (src/duplex/streaming/
 * fused_packed_moe.py:222-263) as that stack runs them.  The blocks: top-8 (one
 * slot per XCD), CT experts, router_w present, H = 1024 or 2048, the shapes of
 * i4_moe_forward's single-launch decode layer.  Slot j's gate_up and down
 * workgroups all run on XCD j; the down workgroups take the slot's activations
 * over through that XCD's L2 and write the slot's output rows, ypart[j][H]
 * (x_dtype, 16-byte aligned), rounded to x_dtype as the reference rounds each
 * expert's output (:262).  The routing-weighted sum is left to the next launch:
 *   i4_moe_route_sum: the router launch of a layer (logits, RMSNorm, as
 *     i4_moe_forward's) on res [H] when ypart is NULL; otherwise it first completes
 *     the previous layer, h = res + sum_j w_j ypart[j] in fp32 in slot order,
 *     rounded once (the arithmetic of i4_moe_forward's combine), writes h to h_out
 *     and routes h.  w_j are the weights the previous i4_moe_experts_x call left in
 *     the workspace.  reset_status = 1 clears the status word.
 *   i4_moe_experts_x: the experts launch of that layer from the logits in the
 *     workspace (every workgroup ranks them itself); it reads RMSNorm(h) from the
 *     workspace, or h when the block has no norm.  down_only = 1 launches the down
 *     workgroups alone: they wait for activations nobody writes, which the bound
 *     max_polls turns into NaN rows and I4_ERR_HANDOFF in the status word (a test
 *     of the bounded wait from the host; the stack passes 2^20).
 *   i4_moe_sum: out = res + sum_j w_j ypart[j], the last layer's completion.
 * The workspace is i4_moe_forward's T = 1 workspace (i4_moe_workspace_bytes(1, H,
 * I, E, 8); the status word at i4_moe_status_offset); calls sharing it run in
 * stream order and must not overlap. */
int    i4_moe_route_sum(const void* res, int x_dtype, const void* ypart,
                        const i4_moe_weights* weights, int topk, void* h_out,
                        int reset_status, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);
int    i4_moe_experts_x(const void* h, int x_dtype, const i4_moe_weights* weights, int topk,
                        int renorm, void* ypart, int max_polls, int down_only,
                        void* workspace, size_t workspace_bytes, hipStream_t stream);
int    i4_moe_sum(const void* res, int x_dtype, const void* ypart,
                  const i4_moe_weights* weights, int topk, void* out,
                  const void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Qwen3OmniMoeThinkerTextRMSNorm.forward (transformers modeling_qwen3_omni_moe.py:
 * 1388-1393, 5.15; the Thinker decoder layer's input_layernorm, which the clock
 * path runs in front of every attention block, clock.py:164-172):
 *   out[t] = w * (x[t] * rsqrt(mean(x[t]^2) + eps)), the normalised row rounded to
 *   x_dtype before the weight multiply, as the reference casts.  H % 8 == 0, H <= 4096. */
int    i4_rmsnorm(const void* x, int x_dtype, int T, int H, const void* norm_w, float eps,
                  void* out, hipStream_t stream);

/* The attention core of one decode token of a Thinker layer,
 * Qwen3OmniMoeThinkerTextAttention.forward (modeling_qwen3_omni_moe.py:1473-1514)
 * between its q/k/v and o projections, with the DynamicCache of clock.py:164-172:
 *   qkv      [n_heads + 2 n_kv_heads][head_dim], the fused q|k|v projection output;
 *   q/k      RMSNorm over head_dim with q_norm_w / k_norm_w, then the rotary
 *            embedding at position pos with inv_freq[head_dim / 2] (host array;
 *            text positions make the interleaved mRoPE the 1-D one);
 *   cache    k_cache / v_cache [n_kv_heads][max_len][head_dim]; row pos receives this
 *            token's k and v, rows [0, pos] are attended (GQA: query head h reads kv
 *            head h / (n_heads / n_kv_heads));
 *   out      [n_heads][head_dim] = softmax(q k^T / sqrt(head_dim)) v, fp32 inside,
 *            rounded once to x_dtype.
 * head_dim == 128, n_heads / n_kv_heads <= 8, 0 <= pos < max_len <= 65536.  The workspace
 * (i4_attn_decode_workspace_bytes) needs no initial contents; calls sharing one must not
 * overlap. */
int    i4_attn_decode(const void* qkv, int x_dtype, int n_heads, int n_kv_heads, int head_dim,
                      const void* q_norm_w, const void* k_norm_w, float eps,
                      const float* inv_freq, int pos, void* k_cache, void* v_cache,
                      int max_len, void* out, void* workspace, size_t workspace_bytes,
                      hipStream_t stream);
/* i4_attn_decode with the position in device memory (int32, read by the kernels), so one
 * captured hipGraph of a decode step serves every token: the launch covers all of max_len's
 * 64-position chunks and those past *pos exit at once.  A *pos outside [0, max_len) writes
 * nothing to the caches and NaN to out. */
int    i4_attn_decode_at(const void* qkv, int x_dtype, int n_heads, int n_kv_heads,
                         int head_dim, const void* q_norm_w, const void* k_norm_w, float eps,
                         const float* inv_freq, const int32_t* pos, void* k_cache,
                         void* v_cache, int max_len, void* out, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);
size_t i4_attn_decode_workspace_bytes(int n_heads, int head_dim, int max_len);
/* The attention core above followed by the o_proj projection with the residual added,
 *   y = residual + o_w attn,   y / residual [o_w->N] in x_dtype (residual nullable),
 * which the reference runs as the attention then TritonPackedLinear(o_proj)
 * (triton_dequant_gemv.py:151-159) and the decoder layer's residual add
 * (modeling_qwen3_omni_moe.py:1547-1552 in transformers 5.15).  o_w: one CT weight
 * (E = 1) with K = n_heads * head_dim <= 8192.  The chunk merge and o_proj run as one
 * launch whose o_proj workgroups stream their weights while the heads are merged and
 * then take the merged heads over inside the launch; the result equals
 * i4_attn_decode(_at) followed by i4_linear(o_w, bias = residual) bit for bit.
 * pos_dev (int32 on the device, nullable) overrides pos as in i4_attn_decode_at.
 * Workspace: i4_attn_decode_o_workspace_bytes(), no initial contents; calls sharing one
 * must not overlap.  Its int32 at i4_attn_decode_o_status_offset() is a status word every
 * call rewrites: I4_OK, or I4_ERR_HANDOFF when an o_proj workgroup gave up waiting for
 * the merged heads of its own launch (its rows are then NaN; the wait is bounded at 2^20
 * polls and only gives up if the launch's workgroups are not dispatched in block order). */
int    i4_attn_decode_o(const void* qkv, int x_dtype, int n_heads, int n_kv_heads,
                        int head_dim, const void* q_norm_w, const void* k_norm_w, float eps,
                        const float* inv_freq, const int32_t* pos_dev, int pos, void* k_cache,
                        void* v_cache, int max_len, const i4_qweight* o_w,
                        const void* residual, void* y, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);
size_t i4_attn_decode_o_workspace_bytes(int n_heads, int head_dim, int max_len);
size_t i4_attn_decode_o_status_offset(int n_heads, int head_dim, int max_len);

/* The attention half of a Thinker decoder layer for one decode token, from the layer's
 * input row h:
 *   y = h + o_w attn(qkv_w rmsnorm(h; in_norm_w, eps)),
 * the first lines of Qwen3OmniMoeThinkerTextDecoderLayer.forward
 * (modeling_qwen3_omni_moe.py:1539-1552 in transformers 5.15) with q_proj / k_proj /
 * v_proj and o_proj on TritonPackedLinear (triton_dequant_gemv.py:151-159).  qkv_w: one
 * CT weight [(n_heads + 2 n_kv_heads) head_dim][H]; o_w: one CT weight [H][n_heads
 * head_dim] (K <= 8192); the other arguments as in i4_attn_decode_o.  Where the q|k|v
 * GEMV has 32 lanes per row and H <= 4096 (the Thinker's 2048 -> 5120), the input norm
 * and the projection run inside the attention chunk launch, whose chunk workgroups take
 * their q / k / v rows over as (value pair, tag) words; two launches in all.  Otherwise
 * three (i4_rmsnorm_linear first).  Either way the result and the cache rows equal
 * i4_rmsnorm_linear + i4_attn_decode_o(residual = h) bit for bit.  h: 16-byte aligned;
 * y may be h.  Workspace: i4_attn_decode_qkv_o_workspace_bytes(), 256-byte aligned, the
 * layout of i4_attn_decode_o's (status word at i4_attn_decode_o_status_offset(), also for
 * a chunk workgroup whose wait for its rows gave up) then the q|k|v row; it needs no
 * initial contents, and one zero-filled at allocation cannot agree with a hand-over tag
 * by chance (the tags are odd); calls sharing one must not overlap. */
int    i4_attn_decode_qkv_o(const void* h, int x_dtype, const void* in_norm_w, float eps,
                            const i4_qweight* qkv_w, int n_heads, int n_kv_heads, int head_dim,
                            const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                            const int32_t* pos_dev, int pos, void* k_cache, void* v_cache,
                            int max_len, const i4_qweight* o_w, void* y, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);
size_t i4_attn_decode_qkv_o_workspace_bytes(int n_heads, int n_kv_heads, int head_dim,
                                            int max_len);

/* One decode token through a whole Thinker decoder layer:
 * Qwen3OmniMoeThinkerTextDecoderLayer.forward (modeling_qwen3_omni_moe.py:1539-1565
 * in transformers 5.15), whose MoE block the reference replaces with
 * FusedPackedMoE.forward (src/duplex/streaming/fused_packed_moe.py:191-220):
 *   h2  = h + o_w attention(RMSNorm(h; in_norm_w, eps) qkv_w^T)
 *   out = h2 + MoE(RMSNorm(h2; moe->norm_w, moe->norm_eps))
 * with the attention of i4_attn_decode_o (q_norm_w / k_norm_w also use eps) and the
 * MoE block of i4_moe_forward at T = 1 (router_w and norm_w required, CT experts).
 * Three launches: the q|k|v GEMV with the input norm inside the attention chunk launch
 * (as in i4_attn_decode_qkv_o; a separate launch first where its shape does not allow),
 * the head merge + o_proj + the MoE router (the router waves wait inside that launch for
 * the o_proj output), the experts.  The result, the cache rows and the MoE status word
 * equal i4_rmsnorm_linear + i4_attn_decode_o(residual = h) + i4_moe_forward(T = 1,
 * residual = h2) bit for bit.  qkv_w, o_w: one CT weight each, qkv_w [(n_heads +
 * 2 n_kv_heads) head_dim][H], o_w [H][n_heads head_dim]; H = 1024 or 2048.  h and
 * out ([H], x_dtype, 16-byte aligned) may be the same buffer.  pos_dev as in
 * i4_attn_decode_o.  Workspace: i4_thinker_layer_workspace_bytes(), no initial
 * contents (zero-filled at allocation rules out any chance agreement with the q|k|v
 * hand-over tags, as for i4_attn_decode_qkv_o), 256-byte aligned; it begins with
 * i4_moe_forward's T = 1 workspace, so a
 * router or expert wait that gave up leaves I4_ERR_HANDOFF at
 * i4_moe_status_offset(1, H, I, E, topk).  Calls sharing one must not overlap.
 * i4_thinker_layer_workspace_bytes returns 0 for sizes the entry does not take
 * (also an expert shape outside its single-launch expert kernel). */
int    i4_thinker_layer_decode(const void* h, int x_dtype, const void* in_norm_w, float eps,
                               const i4_qweight* qkv_w, int n_heads, int n_kv_heads,
                               int head_dim, const void* q_norm_w, const void* k_norm_w,
                               const float* inv_freq, const int32_t* pos_dev, int pos,
                               void* k_cache, void* v_cache, int max_len,
                               const i4_qweight* o_w, const i4_moe_weights* moe, int topk,
                               int renorm, void* out, void* workspace, size_t workspace_bytes,
                               hipStream_t stream);
size_t i4_thinker_layer_workspace_bytes(int n_heads, int n_kv_heads, int head_dim,
                                        int max_len, int H, int I, int E, int topk);

/* One Thinker decoder layer's weights and KV cache, for i4_thinker_decode_step. */
typedef struct i4_thinker_layer {
  const void* in_norm_w;   /* [H] input_layernorm weight, x_dtype */
  const void* q_norm_w;    /* [head_dim] q_norm / k_norm weights, x_dtype */
  const void* k_norm_w;
  void*       k_cache;     /* [n_kv_heads][max_len][head_dim], x_dtype */
  void*       v_cache;
  float       eps;         /* input, q and k RMSNorm epsilon */
  i4_qweight  qkv;         /* CT [(n_heads + 2 n_kv_heads) head_dim][H] */
  i4_qweight  o;           /* CT [H][n_heads head_dim] */
  i4_moe_weights moe;      /* CT experts; router_w and norm_w (post-attention norm) */
} i4_thinker_layer;

/* One decode token through n_layers Thinker decoder layers: the clock path's
 * `th(inputs_embeds=emb, past_key_values=th_kv)` over Thinker[0:n] (src/duplex/
 * streaming/clock.py:164-172), i.e. i4_thinker_layer_decode per layer, h -> out,
 * in one call (the hidden state between layers stays in the workspace).  The
 * result and the caches equal i4_thinker_layer_decode applied layer by layer bit
 * for bit.  Every layer has the same head counts, H, I, E; the checks of all
 * layers come before the first launch.  At H = 2048 with the stack's XCD-local
 * experts launch available (top-8 or less), every layer but the last runs that
 * launch instead of the single-block one (its slot outputs stay in the workspace)
 * and the next layer's q|k|v launch completes them into its input row first, with
 * the single-block combine's arithmetic: the same result bit for bit.
 * Workspace: i4_thinker_decode_step_workspace_bytes(), no initial contents,
 * 256-byte aligned; it begins with i4_moe_forward's T = 1 workspace, whose status
 * word (i4_moe_status_offset(1, H, I, E, topk)) is cleared by the first layer and
 * then holds I4_ERR_HANDOFF if any wait of the step gave up. */
int    i4_thinker_decode_step(const void* h, int x_dtype, const i4_thinker_layer* layers,
                              int n_layers, int n_heads, int n_kv_heads, int head_dim,
                              const float* inv_freq, const int32_t* pos_dev, int pos,
                              int max_len, int topk, int renorm, void* out, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);
size_t i4_thinker_decode_step_workspace_bytes(int n_heads, int n_kv_heads, int head_dim,
                                              int max_len, int H, int I, int E, int topk);

/* ------------------------------------------------------------------------
 * MoE block on 16-bit or int8 experts with a sigmoid-gated shared expert: the
 * Talker's block.  Replaces FusedMoE.forward (src/duplex/streaming/fused_moe.py:
 * 99-141), which itself stands in for transformers'
 * Qwen3OmniMoeTalkerTextSparseMoeBlock.forward (modeling_qwen3_omni_moe.py:
 * 2722-2733, transformers 5.15). */

/* One stacked weight [E][N][K], row-major and densely stacked.  scale == NULL:
 * data holds values in the activation dtype; else data holds int8 q and scale
 * [E][N] (activation dtype) one scale per output row, value = q * scale -- the
 * per-output-channel symmetric int8 of FusedMoE's q8 mode (fused_moe.py:84-94). */
typedef struct i4_dweight {
  const void* data;
  const void* scale;
  int32_t     E, N, K;
} i4_dweight;

/* One MoE block as FusedMoE stores it (fused_moe.py:59-97). */
typedef struct i4_dmoe_weights {
  i4_dweight  gate_up;          /* [E][2I][H]: rows [0,I) gate_proj, [I,2I) up_proj */
  i4_dweight  down;             /* [E][H][I]; same format as gate_up               */
  const void* router_w;         /* [E][H] in the activation dtype; may be NULL when
                                   logits are passed                                */
  i4_dweight  shared_gate_up;   /* [1][2Is][H]; data NULL: no shared expert         */
  i4_dweight  shared_down;      /* [1][H][Is]                                       */
  const void* shared_gate_w;    /* [H] (shared_expert_gate, Linear(H, 1)); NULL: 1 */
} i4_dmoe_weights;

/* out[t] = residual[t] + sum_j w[t][j] * down_e(act_e), e = sel[t][j],
 *          act_e = silu(gate_e(x[t])) * up_e(x[t]) rounded to x_dtype
 *          + sigmoid(shared_gate_w . x[t]) * down_s(silu(gate_s x[t]) * up_s x[t])
 * Routing (fused_moe.py:103-108): logits = router_w x (rounded to x_dtype; or the
 * given [T][E] logits when router_w is NULL), softmax in fp32, top-k (ties to the
 * lower id), renormalised over the k when renorm != 0.  The shared gate's logit and
 * sigmoid are rounded to x_dtype as the 16-bit Linear and sigmoid round them; the
 * rest is fp32 and the output is rounded once.  residual, sel_out and w_out
 * ([T][topk], fp32) are optional.  H % 16 == 0, 16 <= H <= 2048; I, Is multiples
 * of 16, at most 1024 (16-bit) or 2048 (int8); E <= 512; topk <= 8, <= 7 with a
 * shared expert; T <= 65535.  Each token streams its own experts' rows (a
 * decode-shaped kernel; the reference gathers per token as well, fused_moe.py:121). */
int    i4_dmoe_forward(const void* x, int x_dtype, int T, const i4_dmoe_weights* weights,
                       int topk, int renorm, const void* logits, const void* residual,
                       void* out, int32_t* sel_out, float* w_out, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);
/* Workspace of i4_dmoe_forward (logits, routing, activations; 16-byte aligned, no
 * initial contents).  Calls sharing one workspace must not overlap. */
size_t i4_dmoe_workspace_bytes(int T, int E, int topk, int I, int Is);

/* One decode token (T = 1) with router_w in the block and 16-bit routed experts
 * runs in two launches:
 * the router's, which also marks the activations pending, and one launch
 * whose gate|up workgroups write them while its down workgroups rank the
 * logits themselves and poll the activations until no value still holds the
 * pending pattern 0xFFFF (topk * I + Is <= 4096).  Byte offset, in the
 * workspace of i4_dmoe_forward with these sizes, of the int32 status word
 * every call rewrites: I4_OK, or I4_ERR_HANDOFF when a down workgroup gave up
 * waiting (its output row is then NaN).  As for i4_moe_status_offset, the
 * wait assumes block-order dispatch (no reference counterpart). */
size_t i4_dmoe_status_offset(int T, int E, int topk, int I, int Is);

/* The down workgroups of that launch on their own, for one token (T = 1) with
 * the given [E] logits: they poll the workspace's activations as they are,
 * at most max_polls times, and a workgroup that gives up writes NaN to its
 * row and I4_ERR_HANDOFF to the status word (only the failure is stored).
 * 16-bit routed experts.  For testing the bounded wait from the host (the
 * reference's block, fused_moe.py:99-141, has no such wait). */
int    i4_dmoe_down_wait(const void* x, int x_dtype, const i4_dmoe_weights* weights,
                         int topk, int renorm, const void* logits, const void* residual,
                         void* out, void* workspace, size_t workspace_bytes, int max_polls,
                         hipStream_t stream);

/* ------------------------------------------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc): i4_moe_forward with its workspace taken from a static
 * device array of I4_NOALLOC_SCRATCH_BYTES inside the library, one per GPU,
 * held until the process ends.  It allocates nothing and calls no allocating
 * routine.  A call whose i4_moe_workspace_bytes() exceeds the array returns
 * I4_ERR_SCRATCH without launching (8 MiB covers a decode token and batches of
 * up to ~160 tokens at hidden 2048, FFN 768, 128 experts, top-8).  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU race.  status_out
 * (int32 on the device, 4-byte aligned, nullable) receives the status word that
 * i4_moe_forward keeps in its workspace: I4_OK, or I4_ERR_HANDOFF when a decode wait
 * gave up (NaN rows); the call rewrites it. */
#define I4_NOALLOC_SCRATCH_BYTES (8u << 20)
int    i4_moe_forward_noalloc(const void* x, int x_dtype, int T,
                              const i4_moe_weights* weights, int topk, int renorm,
                              const void* logits, const void* residual, void* out,
                              int32_t* sel_out, float* w_out, int32_t* status_out,
                              hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* I4MOE_H */
