// Launchers of the MoE kernels (I4_LAYOUT_TILE weights), shared between the
// translation units of libi4moe.  Callers have validated every argument.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "i4_tile.h"

namespace i4 {

static constexpr int MF_TOK = 64;    // tokens per entry of the large-entry MFMA kernel
static constexpr int LIN_TOK = 64;   // rows per tile of the dense linear MFMA launch
static constexpr int ONE_LIST_T = 64;  // up to this many tokens: small entries only
static constexpr int MF_SMALL = 16;  // experts with at most this many tokens: one m-block
static constexpr int MF_NB = 2;      // n-blocks of 16 weight rows per wave

// decode gate_up + SiLU: slot j of token 0 (route: ranked from logits in the
// kernel, sel / wts written for the down stage; else expert sel[j])
struct GateUpArgs {
  bool route;
  int n_slots;  // grid rows: slots computed
  int topk;
  int E_r;      // logits per row (route)
  int renorm;
  const void* x;
  int32_t* sel;
  const void* logits;
  float* wts;
  void* act;
  int32_t* status;  // nullable: workgroup (0, 0) sets it to I4_OK (no wait in these kernels)
};

// tile weights (i4_moe_decode.hip)
template <int XT, int ST>
int launch_gate_up(const GateUpArgs& a, const TW& w, int I, hipStream_t s);
template <int XT, int ST>
int launch_down_m1(const void* act, int topk, const int32_t* sel, const float* wts, const TW& w,
                   const void* residual, void* out, hipStream_t s);
// CT weights (i4_moe_ct.hip); TW carries the CT pointers and strides
template <int XT, int ST>
int launch_gate_up_ct(const GateUpArgs& a, const TW& w, int I, hipStream_t s);
template <int XT, int ST>
int launch_down_m1_ct(const void* act, int topk, const int32_t* sel, const float* wts,
                      const TW& w, const void* residual, void* out, hipStream_t s);
// both expert projections of a decode layer in one launch (route mode only);
// act must hold the pending pattern (kPending16) in its topk * I values, which
// the T = 1 router launch writes.  A down workgroup polls act at most
// max_polls times; one that gives up writes NaN rows and I4_ERR_HANDOFF to
// *status.  gate_up == nullptr launches the down workgroups alone (act is then
// produced elsewhere).  moe_m1_ct_fits says which shapes it covers.
static constexpr int kHandoffPolls = 1 << 20;
bool moe_m1_ct_fits(int topk, int H, int I);
template <int XT, int ST>
int launch_moe_m1_ct(const GateUpArgs& a, const TW* gate_up, const TW& down,
                     const void* residual, void* out, int32_t* status, int max_polls,
                     hipStream_t s);

// The same layer with slot j's gate_up and down workgroups on XCD j (top-8): the
// down workgroups take act[j] over through that XCD's L2 and write the slot's
// output rows ypart[j][H] (activation dtype); the routing-weighted sum and the
// residual are left to the next launch (i4_launch_router_sum / i4_launch_moe_sum,
// with the weights block 0 writes to a.wts).  act must hold the pending pattern.
// down_only launches the down workgroups alone (act is then produced elsewhere).
bool moe_m1x_ct_fits(int topk, int H, int I);
template <int XT, int ST>
int launch_moe_m1x_ct(const GateUpArgs& a, const TW& gate_up, const TW& down, void* ypart,
                      int32_t* status, int max_polls, bool down_only, hipStream_t s);

// The T = 1 MoE block of a decoder layer whose router runs in an earlier launch
// (i4_thinker_layer_decode, i4_attn.hip): that launch writes the logits and the
// normalised row, arms act with the pending pattern and reports a wait that gave
// up in status; the buffers are those of i4_moe_forward's T = 1 workspace at ws.
struct MoeDecodeBufs {
  uint16_t* logits;  // [E] router logits, the activation dtype
  uint16_t* xn;      // [H] RMSNorm(x) with the block's norm weight
  u32x4* act;        // [topk * I] activations, n_act 16-byte words
  int n_act;
  int32_t* status;
  float* w;          // [topk] routing weights the experts launch writes
  int H, I, E;
  i4_qweight gate_up, down;  // validated (i4_check_weight) CT weights
};
// Validates the block for that use (CT rows, router and norm present, a shape of
// the single-launch expert kernel, H the router wave's 1024 or 2048).
int moe_decode_bufs(const i4_moe_weights* mw, int x_dtype, int topk, void* ws, size_t ws_bytes,
                    MoeDecodeBufs* b);
// The experts launch of that block: out = residual + MoE(xn) from the logits.
int moe_decode_experts(const MoeDecodeBufs& b, int x_dtype, int topk, int renorm,
                       const void* residual, void* out, void* ws, hipStream_t s);
// The XCD-local experts launch of that block (moe_m1x_ct_fits): the slot outputs to
// ypart [topk][H] and the routing weights to b.w; a later launch completes the layer,
// residual + sum_k w[k] ypart[k] (slot_sum8).
int moe_decode_experts_x(const MoeDecodeBufs& b, int x_dtype, int topk, int renorm, void* ypart,
                         void* ws, hipStream_t s);

// Grouped (T > 1) expert projections on MFMA.  entries[i] = {expert, first
// position, tokens, 0} of the expert-sorted (token, slot) list perm; small
// entries have <= MF_SMALL tokens, large ones <= MF_TOK.
//   gate_up: act[pos] = silu(gate(x[perm[pos] / topk])) * up(...), x [T][H]
//   down:    ys[perm[pos]] = down(act[pos]) rounded to the activation dtype
//            (the reference's y.to(x.dtype), fused_packed_moe.py:262), act [rows][I]
template <int XT, int ST>
int launch_mfma_gate_up(bool small, int max_entries, const void* x, int T, int topk,
                        const int4* ent, const int* nent, const int32_t* perm, const TW& w, int I,
                        void* act, hipStream_t s);
template <int XT, int ST>
int launch_mfma_down(bool small, int max_entries, const void* act, int rows, const int4* ent,
                     const int* nent, const int32_t* perm, const TW& w, void* ys, hipStream_t s);

// Both lists of one projection in one launch over max_large + max_small grid
// rows: the large entries first, the small ones right after them, idle rows
// last.  gate_up: src = x, out = act; down: src = act, out = ys.
template <int XT, int ST>
int launch_mfma_mixed(bool gate_up, int max_large, int max_small, const void* src, int src_rows,
                      int topk, const int4* large, const int* n_large, const int4* small,
                      const int* n_small, const int32_t* perm, const TW& w, int I, void* out,
                      hipStream_t s);

// Both projections of small entries (T <= 64) in one launch: the gate_up workgroups
// first, then the down workgroups, which take act over inside the launch (it must hold
// the pending pattern before it; a wait that gives up leaves NaN rows and
// I4_ERR_HANDOFF in *status).  down_only: the down workgroups alone.
template <int XT, int ST>
int launch_mfma_gd(int max_entries, const void* x, int T, int topk, const int4* ent,
                   const int* nent, const int32_t* perm, const TW& wg, const TW& wd, int I,
                   void* act, void* ys, int32_t* status, int max_polls, bool down_only,
                   hipStream_t s);

// Dense linear layer on MFMA: y[M][N] = x[M][K] W^T (+ bias, dtype ot), W one
// tile-layout weight (E = 1, N % 128 == 0).  Small grids are split along K
// into fp32 partials in ws (linear_tile_workspace_bytes; 0 when not split).
template <int XT, int ST>
int launch_mfma_linear(const void* x, int M, const TW& w, const void* bias, void* y, int ot,
                       void* ws, size_t ws_bytes, hipStream_t s);
size_t linear_tile_workspace_bytes(int M, int N, int K);

}  // namespace i4
