"""Host-side logic of the package (no GPU needed): descriptor validation and
the refusal to run anything off the HIP device."""
from __future__ import annotations

import pytest
import torch


def test_qweight_shape_checks(pkg):
    p = torch.zeros(2, 16, 32, dtype=torch.int32)
    s = torch.zeros(2, 16, 8, dtype=torch.float16)
    w = pkg.QWeight(p, s, None, "ct", 32, 16, 256)
    assert (w.E, w.N, w.K) == (2, 16, 256)
    c = w.c()
    assert (c.E, c.N, c.K, c.group, c.layout, c.scale_dtype) == (2, 16, 256, 32, 0, 1)
    with pytest.raises(ValueError):
        pkg.QWeight(p, s[:, :, :4], None, "ct", 32, 16, 256)
    with pytest.raises(ValueError):
        pkg.QWeight(p.float(), s, None, "ct", 32, 16, 256)
    with pytest.raises(ValueError):
        pkg.QWeight(p, s, None, "gptq", 32, 16, 256)
    qa = torch.zeros(2, 256, 2, dtype=torch.int32)
    sa = torch.zeros(2, 2, 16, dtype=torch.float16)
    za = torch.zeros(2, 2, 2, dtype=torch.int32)
    wa = pkg.QWeight.awq(qa, sa, za, group=128)
    assert (wa.N, wa.K, wa.layout) == (16, 256, "awq")
    # 2-D tensors are one expert
    w1 = pkg.QWeight.ct(p[0], s[0], group=32)
    assert w1.E == 1


def test_ops_refuse_cpu_tensors(pkg):
    x = torch.zeros(256, dtype=torch.float16)
    p = torch.zeros(2, 16, 32, dtype=torch.int32)
    s = torch.zeros(2, 16, 8, dtype=torch.float16)
    sel = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="HIP device"):
        pkg.dequant_gemv(x, p, s, sel)
    with pytest.raises(RuntimeError, match="HIP device"):
        pkg.route(torch.zeros(1, 8), 2)


def test_reference_only_modes_are_rejected(pkg):
    with pytest.raises(NotImplementedError):
        pkg.FusedPackedMoE(None, host_resident=True)
    with pytest.raises(NotImplementedError):
        pkg.fuse_packed_moe_blocks(torch.nn.Linear(2, 2), cpu_compute=True)


def test_library_path_is_in_tree(pkg):
    from qwen3_omni_duplex_amd import _lib

    assert _lib.LIB_PATH.parent.name == "qwen3-omni-duplex_amd"
    assert _lib.LIB_PATH.exists()


def test_shared_qkv_serves_each_slice_once_per_input(pkg):
    """The fused q/k/v launch runs once for the three projections of one input and again for
    a new input, even one that reuses the same memory (its cache is dropped after the third
    slice), an in-place change, or a repeated slice."""
    from qwen3_omni_duplex_amd.linear import _SharedQKV

    calls = []

    def fused(x):
        calls.append(x.clone())
        return (x + 1, x + 2, x + 3)

    sh = _SharedQKV(fused)
    x = torch.zeros(2, 4)
    q, k, v = sh.take(x, 0), sh.take(x, 1), sh.take(x, 2)
    assert len(calls) == 1 and torch.equal(q, x + 1) and torch.equal(v, x + 3)
    # same storage, same version, after all three slices were served: a fresh launch
    sh.take(x, 0)
    assert len(calls) == 2
    # an in-place change between the slices: recomputed from the new values
    x.add_(5)
    k2 = sh.take(x, 1)
    assert len(calls) == 3 and torch.equal(k2, x + 2)
    # the same slice twice without the others: the second call launches again
    sh.take(x, 1)
    assert len(calls) == 4


def test_qweight_uses_expert_strided_views_in_place(pkg):
    """A view that is strided between experts only (e.g. the up half of a stacked gate|up) is
    used in place, its stride carried in the descriptor; a view whose rows are not dense is
    refused instead of being copied behind the caller's back."""
    gu = torch.arange(4 * 32 * 16, dtype=torch.int32).reshape(4, 32, 16)
    sc = torch.ones(4, 32, 4, dtype=torch.float16)
    up = pkg.QWeight(gu[:, 16:], sc[:, 16:], None, "ct", 32, 16, 128)
    assert up.packed.data_ptr() == gu[:, 16:].data_ptr()   # no copy
    c = up.c()
    assert (c.packed_estride, c.scale_estride, c.zeros_estride) == (32 * 16, 32 * 4, 0)
    dense = pkg.QWeight(gu, sc, None, "ct", 32, 32, 128)
    assert dense.c().packed_estride == 32 * 16  # any stride is passed explicitly
    one = pkg.QWeight(gu[1], sc[1], None, "ct", 32, 32, 128)
    assert one.E == 1 and one.c().packed_estride == 0
    with pytest.raises(ValueError, match="densely"):
        pkg.QWeight(gu[:, :, :8], sc[:, :, :2], None, "ct", 32, 32, 64)   # rows cut short
    with pytest.raises(ValueError, match="densely"):
        pkg.QWeight(gu.transpose(1, 2).contiguous().transpose(1, 2), sc, None, "ct", 32, 32, 128)
    with pytest.raises(ValueError, match="densely"):  # experts that overlap in memory
        pkg.QWeight(gu[:1].expand(4, 32, 16), sc, None, "ct", 32, 32, 128)


def test_block_weights_must_match_the_activation_dtype(pkg):
    """The kernels read the router and norm weights in the activation dtype (as the
    reference's half-precision gate Linear does, where F.linear raises on a mismatch)."""
    from qwen3_omni_duplex_amd import ops

    rw = torch.zeros(8, 64, dtype=torch.bfloat16)
    nw = torch.ones(64, dtype=torch.float16)
    ops._check_block_dtypes(torch.bfloat16, 64, 8, rw, None)
    with pytest.raises(RuntimeError, match="router weight is torch.bfloat16"):
        ops._check_block_dtypes(torch.float16, 64, 8, rw, None)
    with pytest.raises(RuntimeError, match="norm weight"):
        ops._check_block_dtypes(torch.bfloat16, 64, 8, rw, nw)
    with pytest.raises(RuntimeError, match=r"\[8, 64\]"):
        ops._check_block_dtypes(torch.bfloat16, 64, 8, rw.t().contiguous().t()[:, :32], None)
    with pytest.raises(RuntimeError, match=r"\[8, 64\]"):
        ops._check_block_dtypes(torch.bfloat16, 64, 8, torch.zeros(16, 64, dtype=torch.bfloat16),
                                None)


def test_concat_cols_awq_keeps_the_awq_format(pkg):
    """q|k|v side by side in AWQ packing: words, scales and zero words concatenated along
    N; a part without zero points gets explicit 8s.  Dequantised by the oracle, the result
    is the parts' rows stacked in order (pins the layout the in-place GEMV reads)."""
    import numpy as np

    from oracle import i4ref
    from tests import _gen

    rng = np.random.default_rng(5)
    K, G = 256, 128
    parts, dense = [], []
    for i, N in enumerate((64, 32, 32)):
        qw, qz, sc = _gen.awq_weight(rng, 1, K, N, G)
        z = None if i == 1 else torch.from_numpy(qz)
        parts.append(pkg.QWeight(torch.from_numpy(qw), torch.from_numpy(sc), z, "awq", G, N, K))
        dense.append(i4ref.awq_dequant(qw[0], None if i == 1 else qz[0], sc[0], G))
    w = pkg.concat_cols_awq(parts)
    assert (w.layout, w.N, w.K, w.E) == ("awq", 128, K, 1)
    assert torch.equal(w.packed[0, :, 8:12], parts[1].packed[0])
    assert (w.zeros[0, :, 8:12] == -2004318072).all()  # 0x88888888: every zero point 8
    got = i4ref.awq_dequant(w.packed[0].numpy(), w.zeros[0].numpy(), w.scale[0].numpy(), G)
    assert np.array_equal(got, np.concatenate(dense, axis=0))
    qw, qz, sc = _gen.awq_weight(rng, 1, 128, 32, G)  # another K
    other = pkg.QWeight(torch.from_numpy(qw), torch.from_numpy(sc), torch.from_numpy(qz), "awq",
                        G, 32, 128)
    with pytest.raises(ValueError):
        pkg.concat_cols_awq([parts[0], other])

