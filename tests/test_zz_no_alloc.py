"""i4_moe_forward_noalloc (the library's static per-GPU scratch instead of a workspace)
against i4_moe_forward on the same inputs, through the C ABI: bit for bit, on two calls in a
row with the second smaller, at decode (the single-launch layer) and in a batch (the grouped
MFMA path); a call beyond the scratch is refused without launching."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.test_gpu_parity import _awq_moe, make_x, t_

pytestmark = pytest.mark.gpu
H, I, K8 = 2048, 768, 8


def _both(pkg, moe, x, res):
    kw = dict(router_w=moe.router_w, residual=res, gate_up_tile=moe.gate_up_tile,
              down_tile=moe.down_tile)
    want = pkg.moe_forward(x, moe.gate_up, moe.down, K8, **kw)
    status = torch.full((1,), 12345, dtype=torch.int32, device=x.device)
    got = pkg.moe_forward_noalloc(x, moe.gate_up, moe.down, K8, status=status, **kw)
    torch.cuda.synchronize()
    assert int(status.item()) == 0  # the call rewrites the caller's status word
    return got, want


def test_noalloc_matches_the_workspace_entry_point(pkg, dev):
    rng = np.random.default_rng(201)
    moe, _, _, _ = _awq_moe(pkg, dev, rng)
    for T in (48, 1, 32, 1):  # each call after the first is smaller than the one before
        x = t_(make_x(rng, (T, H), "f16"), dev)
        res = t_(make_x(rng, (T, H), "f16"), dev)
        got, want = _both(pkg, moe, x, res)
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), f"T={T}"
    lib = pkg.lib()
    big = lib.i4_moe_workspace_bytes(1024, H, I, 128, K8)
    assert big > (8 << 20)
    x = t_(make_x(rng, (1024, H), "f16"), dev)
    with pytest.raises(RuntimeError, match="static buffer"):
        pkg.moe_forward_noalloc(x, moe.gate_up, moe.down, K8, router_w=moe.router_w,
                                gate_up_tile=moe.gate_up_tile, down_tile=moe.down_tile)


def test_noalloc_logits_and_norm(pkg, dev):
    """Routing from given logits, and the fused pre-MoE RMSNorm, through the static scratch."""
    rng = np.random.default_rng(202)
    moe, _, _, _ = _awq_moe(pkg, dev, rng, E=64)
    nw = t_(rng.uniform(0.5, 1.5, H).astype(np.float16), dev)
    for T in (5, 1):
        x = t_(make_x(rng, (T, H), "f16"), dev)
        lg = t_(rng.standard_normal((T, 64)).astype(np.float16), dev)
        tiles = dict(gate_up_tile=moe.gate_up_tile, down_tile=moe.down_tile)
        want = pkg.moe_forward(x, moe.gate_up, moe.down, K8, logits=lg, **tiles)
        got = pkg.moe_forward_noalloc(x, moe.gate_up, moe.down, K8, logits=lg, **tiles)
        assert torch.equal(got, want)
        want = pkg.moe_forward(x, moe.gate_up, moe.down, K8, router_w=moe.router_w, norm_w=nw,
                               residual=x, **tiles)
        got = pkg.moe_forward_noalloc(x, moe.gate_up, moe.down, K8, router_w=moe.router_w,
                                      norm_w=nw, residual=x, **tiles)
        assert torch.equal(got, want)
