"""ccq_moe_w4_forward_noalloc (the MoE layer from router logits with its
workspace in the library's per-GPU scratch array) against
ccq_moe_w4_forward with a caller workspace: the same kernels, so routing
ids, weights and the output agree bit for bit.  Two calls in a row, the
second on a smaller batch (the array keeps the first call's contents), then
a batch too large for the array, rejected on the host."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import awq as oawq

pytestmark = pytest.mark.gpu


def _layer(gpu, E, H, I, G, seed):
    from ccut.blocks import moe

    rng = np.random.default_rng(seed)

    def one(K, N):
        q = rng.integers(0, 16, size=(E, K, N), dtype=np.uint8)
        z = rng.integers(0, 16, size=(E, K // G, N), dtype=np.uint8)
        s = (np.abs(rng.standard_normal((E, K // G, N))) * 0.01 + 1e-3).astype(np.float16)
        return tuple(torch.from_numpy(a).to(gpu) for a in
                     (np.stack([oawq.pack(a) for a in q]), np.stack([oawq.pack(a) for a in z]), s))

    return moe.W4Experts.from_awq(one(H, I), one(H, I), one(I, H), group_size=G)


def _call(lib, ex, x, lg, k, with_workspace: bool):
    from ccut import _dev
    from ccut._lib import CCQ_BF16, CCQ_F32

    T = x.shape[0]
    y = torch.full((T, ex.hidden), float("nan"), dtype=torch.float32, device=x.device)
    ids = torch.full((T, k), -7, dtype=torch.int64, device=x.device)
    w = torch.full((T, k), float("nan"), dtype=torch.float32, device=x.device)
    desc = ex.descriptor()
    st = _dev.stream_ptr(x.device)
    if with_workspace:
        nbytes = lib.ccq_moe_w4_workspace_size(T, k, ctypes.byref(desc))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        rc = lib.ccq_moe_w4_forward(x.data_ptr(), CCQ_BF16, lg.data_ptr(), T, k, 1, ids.data_ptr(), w.data_ptr(),
                                    y.data_ptr(), CCQ_F32, ctypes.byref(desc), ws.data_ptr(), nbytes, st)
    else:
        rc = lib.ccq_moe_w4_forward_noalloc(x.data_ptr(), CCQ_BF16, lg.data_ptr(), T, k, 1, ids.data_ptr(),
                                            w.data_ptr(), y.data_ptr(), CCQ_F32, ctypes.byref(desc), st)
    return rc, y, ids, w


@pytest.mark.parametrize("E,H,I,k,T1,T2", [(64, 2048, 1408, 6, 16, 3), (8, 256, 384, 2, 200, 40)])
def test_noalloc_matches_workspace_entry(gpu, E, H, I, k, T1, T2):
    """The 64-expert decode layer routes inside the gate/up kernel; E=8 with
    T=200 takes the routing kernel and the grouped prefill kernels."""
    from ccut import _lib

    lib = _lib.lib()
    ex = _layer(gpu, E, H, I, 128, seed=E + T1)
    g = torch.Generator().manual_seed(T1)
    for T in (T1, T2):  # the second call is smaller: stale scratch must not leak into it
        x = torch.randn((T, H), generator=g).to(torch.bfloat16).to(gpu)
        lg = torch.randn((T, E), generator=g).to(gpu)
        rc_a, y_a, ids_a, w_a = _call(lib, ex, x, lg, k, with_workspace=False)
        assert rc_a == 0, _lib.last_error()
        rc_b, y_b, ids_b, w_b = _call(lib, ex, x, lg, k, with_workspace=True)
        assert rc_b == 0, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(ids_a, ids_b)
        assert torch.equal(w_a.view(torch.int32), w_b.view(torch.int32))
        assert torch.equal(y_a.view(torch.int32), y_b.view(torch.int32)), f"T={T}"
        assert torch.isfinite(y_a).all()


def test_noalloc_rejects_batches_beyond_the_array(gpu):
    from ccut import _lib

    lib = _lib.lib()
    ex = _layer(gpu, 64, 2048, 1408, 128, seed=1)
    desc = ex.descriptor()
    T, k = 4096, 6
    assert lib.ccq_moe_w4_workspace_size(T, k, ctypes.byref(desc)) > _lib.CCQ_MOE_W4_NOALLOC_BYTES
    x = torch.zeros((T, 2048), dtype=torch.bfloat16, device=gpu)
    lg = torch.zeros((T, 64), dtype=torch.float32, device=gpu)
    rc, _, _, _ = _call(lib, ex, x, lg, k, with_workspace=False)
    assert rc == _lib.CCQ_EINVAL
    assert "scratch" in _lib.last_error()
