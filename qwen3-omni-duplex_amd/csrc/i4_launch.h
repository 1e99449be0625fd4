// Host-side helpers shared between the translation units of libi4moe.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "i4moe.h"

// log2(group) - 5: group index of 32-column chunk c is c >> shift
inline int i4_group_shift(int group) {
  int sh = 0;
  while ((32 << sh) < group) ++sh;
  return sh;
}

// Validate a weight descriptor; on success *norm holds a copy whose zero
// expert strides are replaced by the dense ones.
int i4_check_weight(const i4_qweight* w, i4_qweight* norm);

// Launch the CT dequant-GEMV: out[j][n] = W[sel[j] or 0] x[j*x_stride] (+bias).
int i4_launch_gemv_ct(const void* x, int xt, int64_t x_stride, const i4_qweight* w,
                      const int32_t* sel, int k_sel, void* out, int ot, const void* bias,
                      hipStream_t s);

// Launch router logits / top-k without re-validating (callers validated).
// T = 1 only: pend (16-byte aligned, n_pend 16-byte units) is filled with
// 0xFFFF halves, the pending pattern of the single-launch expert stage, and
// *status (nullable) is set to I4_OK for the failure that stage may report.
int i4_launch_router_logits(const void* x, int xt, int T, int H, const void* wr, int E,
                            const void* norm_w, float eps, void* xn, void* logits, hipStream_t s,
                            void* pend = nullptr, int n_pend = 0, int32_t* status = nullptr);
// pend (16-byte aligned, n_pend 16-byte units, nullable) is filled with the pending
// pattern for the fused grouped launch after it (k_tile_mfma_gd).
int i4_launch_topk(const void* logits, int lt, int T, int E, int topk, int renorm, int32_t* sel,
                   float* wf, void* wh, int wht, hipStream_t s, void* pend = nullptr,
                   int n_pend = 0);
// Router logits and top-k of 2..64 tokens in one launch (k_router_topk_t; E <= 128,
// E % 4 == 0, else I4_ERR_SHAPE): lgt holds T E 4 bytes of (value pair, tag) words, epoch
// the workspace word a later launch of the call advances (k_group); the routing goes to
// sel / wf, pend as in i4_launch_topk; a ranking wave that gave up writes NaN weights and
// I4_ERR_HANDOFF to *status; status_reset (nullable) is set to I4_OK first.  rank_only:
// the ranking waves alone (their waits give up), for testing the bound.
int i4_launch_router_topk(const void* x, int xt, int T, int H, const void* wr, int E,
                          const void* norm_w, float eps, void* xn, uint32_t* lgt,
                          const uint32_t* epoch, int topk, int renorm, int32_t* sel, float* wf,
                          void* pend, int n_pend, int32_t* status_reset, int32_t* status,
                          int max_polls, bool rank_only, hipStream_t s);

// T = 1 router launch that first completes the previous layer of an XCD-local experts
// launch: h = res + sum_k wts[k] ypart[k] (kc == 8 slot rows of H values), written to
// h_out, then routed as i4_launch_router_logits routes x (H = 1024 or 2048).
int i4_launch_router_sum(const void* res, const void* ypart, const float* wts, int kc,
                         void* h_out, int xt, int H, const void* wr, int E, const void* norm_w,
                         float eps, void* xn, void* logits, hipStream_t s, void* pend,
                         int n_pend, int32_t* status);
// The completion alone: out = res + sum_k wts[k] ypart[k].
int i4_launch_moe_sum(const void* res, const void* ypart, const float* wts, int kc, int xt,
                      int H, void* out, hipStream_t s);

namespace i4 {
// i4_moe_forward with its status word at `status` (device, 4-byte aligned; nullptr: in
// the workspace), for i4_moe_forward_noalloc's status output
int moe_forward_status(const void* x, int x_dtype, int T, const i4_moe_weights* weights,
                       int topk, int renorm, const void* logits, const void* residual, void* out,
                       int32_t* sel_out, float* w_out, void* workspace, size_t workspace_bytes,
                       int32_t* status, hipStream_t stream);
}  // namespace i4
