"""MoE experts in the reference checkpoint's own format -- FP8 e4m3 [out, in]
with one BF16 scale per output row, as ``ExpertReader._fill`` reads them
(reference python/ccut/experts/reader.py:142-251) -- on the fused kernels
(``ccq_moe_fp8row_ffn``): against the oracle's per-row dequant
(``fp8_dequant_mat``, quant/kernels.py:150-171) + ``expert_ffn`` +
``moe_combine`` (blocks/moe.py:122-174), and ``ExpertPipeline.step``
(experts/pipeline.py:123-204) over a safetensors checkpoint at the Ornith
shapes: 256 experts, top-8, hidden 2048, expert intermediate 512.

Tolerances: the kernels' products are exact (weights decoded to bf16, the
float32 activations split into bf16 hi + lo) and accumulate in float32, so
the outputs differ from the float32 reference by summation order only;
the tests assert max|dy| <= 1e-4 * max|y_ref|, tighter than the 2e-2
contract."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle import ref_quant as orq

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _codes(rng, shape):
    """e4m3 codes of moderate magnitude: bit 6 cleared keeps the exponent
    field <= 7 (|value| < 2) and rules out NaN."""
    return (rng.integers(0, 256, size=shape, dtype=np.uint8) & np.uint8(0xBF)).astype(np.uint8)


def _scales(rng, shape):
    s = (np.abs(rng.standard_normal(shape)) * 0.02 + 1e-3).astype(np.float32)
    return torch.from_numpy(s).to(torch.bfloat16).float().numpy()  # BF16 as the checkpoint stores them


def _layer(E, H, I, seed):
    rng = np.random.default_rng(seed)
    return {p: (_codes(rng, (E, o, i)), _scales(rng, (E, o))) for p, (o, i) in
            (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}


def _oracle(x, ids, w, lay, tokens=None):
    """The reference's per-expert path on the oracle: per-row dequant to
    float32 [out, in], transposed to expert_ffn's [in, out], moe_combine."""
    cache = {}

    def lookup(e):
        if e not in cache:
            cache[e] = tuple(orq.fp8_dequant_mat(lay[p][0][e], lay[p][1][e]).T.copy()
                             for p in ("gate", "up", "down"))
        return cache[e]

    if tokens is not None:
        x, ids, w = x[tokens], ids[tokens], w[tokens]
    return omoe.moe_combine(x, ids, w, lookup)


def _experts(lay, gpu):
    from ccut.blocks import moe

    def t(p):
        return (torch.from_numpy(lay[p][0]).to(gpu), torch.from_numpy(lay[p][1]).to(gpu))

    return moe.Fp8RowExperts.from_rows(t("gate"), t("up"), t("down"))


# (E, H, I, T, k): 16-row tiles with 32-column blocks in both stages
# (H, I multiples of 512), 16-column gate/up blocks over 1024-k chunks
# (H a multiple of 1024, a tiny batch), 16-row tiles with 64-column blocks,
# 32- and 64-row tiles, ragged expert loads
CASES = [(8, 512, 512, 3, 2), (8, 1024, 256, 2, 2), (8, 256, 256, 5, 2), (4, 256, 512, 40, 2),
         (4, 512, 256, 64, 2), (6, 256, 256, 37, 3)]


@pytest.mark.parametrize("E,H,I,T,k", CASES)
def test_fp8row_ffn_vs_oracle(gpu, E, H, I, T, k):
    from ccut.blocks import moe

    lay = _layer(E, H, I, seed=E * 1000 + T)
    rng = np.random.default_rng(T)
    x = rng.standard_normal((T, H)).astype(np.float32)
    w, ids = omoe.topk_softmax(rng.standard_normal((T, E)).astype(np.float32), k)
    ex = _experts(lay, gpu)
    y = moe.moe_ffn_fp8row(torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu),
                           torch.from_numpy(w).to(gpu), ex).cpu().numpy()
    ref = _oracle(x, ids, w, lay)
    err = np.abs(y - ref).max() / np.abs(ref).max()
    print(f"fp8row E={E} H={H} I={I} T={T} k={k}: rel err {err:.3e}")
    assert err <= TOL


def test_fp8row_ffn_shared_dropped_and_bf16_out(gpu):
    """The shared expert's add in the combine, an assignment outside [0, E)
    left out, and a bfloat16 output."""
    from ccut.blocks import moe

    E, H, I, T, k = 8, 256, 256, 9, 2
    lay = _layer(E, H, I, seed=77)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((T, H)).astype(np.float32)
    w, ids = omoe.topk_softmax(rng.standard_normal((T, E)).astype(np.float32), k)
    ids_dropped = ids.copy()
    ids_dropped[3, 1] = -1
    shared = rng.standard_normal((T, H)).astype(np.float32)
    ex = _experts(lay, gpu)
    y = moe.moe_ffn_fp8row(torch.from_numpy(x).to(gpu), torch.from_numpy(ids_dropped).to(gpu),
                           torch.from_numpy(w).to(gpu), ex, shared=torch.from_numpy(shared).to(gpu),
                           shared_gate=0.25).cpu().numpy()
    w_kept = np.where(ids_dropped >= 0, w, 0).astype(np.float32)
    unused = ids_dropped.copy()  # the oracle finds a slot by the first match: no repeated ids in a row
    unused[3, 1] = min(set(range(E)) - set(ids[3].tolist()))
    ref = _oracle(x, unused, w_kept, lay) + np.float32(0.25) * shared
    assert np.abs(y - ref).max() <= TOL * np.abs(ref).max()
    yb = moe.moe_ffn_fp8row(torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu),
                            ex, out_dtype=torch.bfloat16).float().cpu().numpy()
    refb = _oracle(x, ids, w, lay)
    assert np.abs(yb - refb).max() <= 1e-2 * np.abs(refb).max()


@pytest.fixture(scope="module")
def ornith_ckpt(tmp_path_factory):
    """One MoE layer in the Ornith checkpoint layout: 256 experts, gate/up
    F8_E4M3 [512, 2048] and down [2048, 512] with BF16 [out, 1] scales under
    ``model.layers.0.mlp.experts.{e}.{proj}_proj.weight`` / ``.weight_scale``
    in two safetensors shards (768 MiB of codes)."""
    from _ckpt import _save

    E, H, I = 256, 2048, 512
    lay = _layer(E, H, I, seed=2026)
    shards = [{}, {}]
    for e in range(E):
        for p in ("gate", "up", "down"):
            name = f"model.layers.0.mlp.experts.{e}.{p}_proj"
            shards[e % 2][name + ".weight"] = torch.from_numpy(lay[p][0][e]).view(torch.float8_e4m3fn)
            shards[e % 2][name + ".weight_scale"] = torch.from_numpy(lay[p][1][e][:, None]).to(torch.bfloat16)
    d = tmp_path_factory.mktemp("ornith")
    _save(d, shards, None)
    return d, lay


@pytest.mark.parametrize("T", [1, 16, 512])
def test_pipeline_ornith_shapes(gpu, ornith_ckpt, T):
    """ExpertPipeline.step over the checkpoint: the reader hands the layer
    over as Fp8RowExperts and the step runs the fused kernels; routing ids
    bit-exact with the oracle's top-k on the same logits; y against the
    oracle's per-row dequant + moe_combine (all tokens up to 16, 48 of the
    512 otherwise: tokens are independent)."""
    from ccut.blocks import moe
    from ccut.experts import ExpertPipeline, ExpertReader, build_expert_index

    path, lay = ornith_ckpt
    E, H, k = 256, 2048, 8
    idx = build_expert_index(path, "model.layers.{layer}.mlp.experts.{expert}.{proj}_proj", num_layers=1,
                             num_experts=E)
    r = ExpertReader(idx, path, num_layers=1)
    rng = np.random.default_rng(100 + T)
    x = rng.standard_normal((T, H)).astype(np.float32)
    gate_w = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    try:
        assert isinstance(r.experts(0), moe.Fp8RowExperts)
        pipe = ExpertPipeline(r)
        y = pipe.step(0, x, gate_w, top_k=k)
        logits = pipe.router_logits(x, gate_w)
    finally:
        r.close()
    logits = logits.cpu().numpy() if isinstance(logits, torch.Tensor) else logits
    w0, ids0 = omoe.topk_softmax(logits, k)
    tokens = np.arange(T) if T <= 16 else np.sort(np.random.default_rng(7).choice(T, 48, replace=False))
    ref = _oracle(x, ids0, w0, lay, tokens)
    err = np.abs(y[tokens] - ref).max() / np.abs(ref).max()
    print(f"ornith pipeline T={T}: rel err {err:.3e}, {len(np.unique(ids0))} experts routed")
    assert y.shape == (T, H) and err <= TOL
    assert pipe.metrics.steps == 1
