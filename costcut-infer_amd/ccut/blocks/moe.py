"""MoE routing and the expert FFN on the GPU (same API as the reference's
``python/ccut/blocks/moe.py``), plus the fused quantized expert forward.

Data flow (reference ``blocks/moe.py:1-15``)::

    logits = router(x)                         # [T, E]
    w, ids = topk_softmax(logits, k)           # ccq_topk_softmax
    schedule = align(ids)                      # ccq_moe_align: experts in
                                               # first-appearance order
    h_e = down_e(silu(gate_e(x)) * up_e(x))    # grouped dequant-GEMM kernels
    y[t] = sum_s w[t, s] * h_{ids[t,s]}[t]     # ccq_moe_combine

The reference-API functions take numpy (returning numpy, as the reference)
or CUDA tensors (staying on the device).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from ccut import _dev
from ccut._lib import call, ccq_fp8_experts, ccq_fp8row_experts, ccq_w4_experts, lib
from ccut.quant import awq

__all__ = [
    "topk_softmax",
    "topk",
    "route_experts",
    "expert_ffn",
    "moe_combine",
    "shared_expert_add",
    "moe_align",
    "W4Experts",
    "moe_forward_w4",
    "Fp8Experts",
    "moe_forward_fp8",
    "Fp8RowExperts",
    "moe_ffn_fp8row",
]

_MODE_SOFTMAX_ALL, _MODE_TOPK_THEN_SOFTMAX, _MODE_RAW_EXP, _MODE_PLAIN, _MODE_ROUTE_NORM = 0, 1, 2, 3, 4


def _route(logits, k: int, mode: int):
    lg = _dev.to_device(logits, torch.float32)
    if lg.dim() != 2:
        raise ValueError(f"router logits must be [T, E], got {tuple(lg.shape)}")
    T, E = lg.shape
    w = torch.empty((T, k), dtype=torch.float32, device=lg.device)
    ids = torch.empty((T, k), dtype=torch.int64, device=lg.device)
    call("ccq_topk_softmax", lg.data_ptr(), w.data_ptr(), ids.data_ptr(), T, E, k, mode, _dev.stream_ptr())
    if _dev.is_host(logits):
        return _dev.to_host(w), _dev.to_host(ids)
    return w, ids


def topk(x, k: int):
    """Per row top-k (values descending, ties to the lowest index), returns
    ``(vals [rows, k], idx [rows, k] int64)`` (reference ``moe.py:46-68``)."""
    vals, idx = _route(x, k, _MODE_PLAIN)
    if isinstance(x, np.ndarray):
        vals = vals.astype(x.dtype, copy=False)
    return vals, idx


def topk_softmax(logits, k: int, norm_topk_prob: bool = True):
    """Routing weights (reference ``moe.py:71-89``): ``norm_topk_prob`` ->
    softmax over the k largest logits; otherwise global softmax, then the k
    largest probabilities (not renormalised)."""
    return _route(logits, k, _MODE_TOPK_THEN_SOFTMAX if norm_topk_prob else _MODE_SOFTMAX_ALL)


def route_experts(gate_logits, top_k: int, norm_topk: int):
    """Fused top-k + softmax (reference ``moe.py:92-119``); ``norm_topk=0``
    normalises exp of the raw selected logits (it disagrees with
    ``topk_softmax(norm_topk_prob=False)`` as in the reference)."""
    return _route(gate_logits, top_k, _MODE_ROUTE_NORM if norm_topk else _MODE_RAW_EXP)


def _f32_weight(w) -> torch.Tensor:
    """A float32 weight on the device, contiguous and 16-byte aligned (the
    fp32 GEMM kernels' 16-byte loads)."""
    t = _dev.to_device(w, torch.float32).contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _expert_shapes(H: int, wg: torch.Tensor, wu: torch.Tensor, wd: torch.Tensor, what: str) -> int:
    I = wg.shape[1] if wg.dim() == 2 else -1
    if wg.dim() != 2 or tuple(wg.shape) != (H, I) or tuple(wu.shape) != (H, I) or tuple(wd.shape) != (I, H):
        raise ValueError(f"{what}: expert weights gate {tuple(wg.shape)}, up {tuple(wu.shape)}, down "
                         f"{tuple(wd.shape)}; expected gate/up [hidden={H}, inter] and down [inter, hidden={H}]")
    return I


def expert_ffn(x, w_gate, w_up, w_down):
    """``down(silu(x @ Wg) * (x @ Wu))`` on already-dequantized float32
    weights ``Wg, Wu [hidden, inter]``, ``Wd [inter, hidden]`` (reference
    ``moe.py:122-141``): ``ccq_expert_ffn_f32``, float32 products on the
    fp32 matrix cores, the SiLU product in float64 (two launches)."""
    xd = _dev.to_device(x, torch.float32).contiguous()
    if xd.dim() != 2:
        raise ValueError(f"x must be [rows, hidden], got {tuple(xd.shape)}")
    rows, H = xd.shape
    wg, wu, wd = _f32_weight(w_gate), _f32_weight(w_up), _f32_weight(w_down)
    I = _expert_shapes(H, wg, wu, wd, "expert_ffn")
    y = torch.empty((rows, H), dtype=torch.float32, device=xd.device)
    if rows:
        nbytes = lib().ccq_expert_ffn_f32_workspace_size(rows, I)
        ws = _dev.workspace("expert_ffn_f32", nbytes, xd.device)
        call("ccq_expert_ffn_f32", xd.data_ptr(), wg.data_ptr(), wu.data_ptr(), wd.data_ptr(), y.data_ptr(), rows,
             H, I, ws.data_ptr(), nbytes, _dev.stream_ptr(xd.device))
    return _dev.to_host(y) if _dev.is_host(x) else y


@dataclass
class Schedule:
    """Expert-sorted tile schedule produced by ``ccq_moe_align``."""

    sorted_ids: torch.Tensor   # [max_tiles * tile_m] int32, -1 = padding
    tile_expert: torch.Tensor  # [max_tiles] int32
    meta: torch.Tensor         # [2] int32: tiles, distinct experts
    counts: torch.Tensor       # [E] int32
    tile_m: int

    def host(self) -> dict:
        nt = int(self.meta[0].item())
        return {
            "num_tiles": nt,
            "num_experts_active": int(self.meta[1].item()),
            "sorted_ids": self.sorted_ids[: nt * self.tile_m].cpu().numpy(),
            "tile_expert": self.tile_expert[:nt].cpu().numpy(),
            "counts": self.counts.cpu().numpy(),
        }


def moe_align(expert_ids, num_experts: int, tile_m: int = 16) -> Schedule:
    """Group the T*k assignments by expert (first-appearance order, tokens
    ascending), padded to ``tile_m`` -- the permutation of the reference's
    ``moe_combine`` (``moe.py:163-167``)."""
    ids = _dev.to_device(expert_ids, torch.int64).reshape(-1)
    n = ids.numel()
    mt = max(1, lib().ccq_moe_align_max_tiles(n, num_experts, tile_m))
    dev = ids.device
    sch = Schedule(torch.empty(mt * tile_m, dtype=torch.int32, device=dev),
                   torch.empty(mt, dtype=torch.int32, device=dev),
                   torch.zeros(2, dtype=torch.int32, device=dev),
                   torch.empty(num_experts, dtype=torch.int32, device=dev), tile_m)
    call("ccq_moe_align", ids.data_ptr(), n, num_experts, tile_m, sch.sorted_ids.data_ptr(),
         sch.tile_expert.data_ptr(), sch.meta.data_ptr(), sch.counts.data_ptr(), _dev.stream_ptr())
    return sch


def moe_combine(x, expert_ids, weights, expert_outputs=None, expert_fn=expert_ffn, w_lookup=None, *,
                shared=None, shared_gate: float = 1.0):
    """``y[t] = sum_e w[t,e] * expert_e(x[t])`` with the tokens of each expert
    batched (reference ``moe.py:144-174``).  With the default ``expert_fn``
    and a ``w_lookup`` returning float32 ``(w_gate, w_up, w_down)``, the
    whole layer is one grouped call (``ccq_moe_f32_ffn``: align, grouped
    gate/up + SiLU, grouped down, combine); with another ``expert_fn``, the
    grouping is computed on the GPU and ``expert_fn`` is called once per
    expert, in first-appearance order, with that expert's rows, and the
    weighted sum is ``ccq_moe_combine``.  ``expert_outputs`` is accepted for
    signature compatibility (the reference ignores it too).  Negative ids
    contribute nothing."""
    xd = _dev.to_device(x, torch.float32).contiguous()
    ids = _dev.to_device(expert_ids, torch.int64).contiguous()
    wts = _dev.to_device(weights, torch.float32).contiguous()
    T, H = xd.shape
    k = ids.shape[1]
    if expert_fn is expert_ffn and w_lookup is not None:
        out = _moe_combine_f32(xd, ids, wts, w_lookup, shared, shared_gate)
        return _dev.to_host(out) if _dev.is_host(x) else out
    E = int(ids.max().item()) + 1 if ids.numel() else 1
    sch = moe_align(ids, max(E, 1), tile_m=1).host()
    rows = torch.zeros((T * k, H), dtype=torch.float32, device=xd.device)
    flat = sch["sorted_ids"]
    pos = 0
    for eid in _experts_in_order(sch):
        cnt = int(sch["counts"][eid])
        a = torch.from_numpy(flat[pos: pos + cnt].astype(np.int64)).to(xd.device)
        pos += cnt
        wg, wu, wd = w_lookup(eid)
        y = expert_fn(xd[a // k], wg, wu, wd)
        rows[a] = _dev.to_device(y, torch.float32)
    out = torch.empty((T, H), dtype=torch.float32, device=xd.device)
    if shared is not None:
        sd = _shared_rows(shared, T, H, xd.device)
        call("ccq_moe_combine_shared", rows.data_ptr(), wts.data_ptr(), sd.data_ptr(), float(np.float32(shared_gate)),
             out.data_ptr(), 0, T, k, H, _dev.stream_ptr())
    else:
        call("ccq_moe_combine", rows.data_ptr(), wts.data_ptr(), out.data_ptr(), 0, T, k, H, _dev.stream_ptr())
    return _dev.to_host(out) if _dev.is_host(x) else out


def _moe_combine_f32(xd: torch.Tensor, ids: torch.Tensor, wts: torch.Tensor, w_lookup, shared,
                     shared_gate: float) -> torch.Tensor:
    """moe_combine's expert_ffn over float32 experts in one grouped call
    (``ccq_moe_f32_ffn``): each routed expert's weights are looked up once,
    and the kernels find them through device tables of pointers."""
    T, H = xd.shape
    k = ids.shape[1]
    out = torch.empty((T, H), dtype=torch.float32, device=xd.device)
    ids_h = ids.cpu().numpy()
    routed = sorted(int(e) for e in np.unique(ids_h) if e >= 0)
    if not routed:
        out.zero_()
        if shared is not None:
            shared_expert_add(out, shared, shared_gate)
        return out
    E = routed[-1] + 1
    keep, tabs, I = [], [[0] * E for _ in range(3)], None
    for e in routed:
        wg, wu, wd = (_f32_weight(w) for w in w_lookup(e))
        Ie = _expert_shapes(H, wg, wu, wd, f"w_lookup({e})")
        if I is not None and Ie != I:
            raise ValueError(f"w_lookup({e}): inter={Ie}, other experts have {I}")
        I = Ie
        keep.append((wg, wu, wd))
        for t, w in zip(tabs, (wg, wu, wd)):
            t[e] = w.data_ptr()
    tab = torch.tensor(tabs, dtype=torch.int64).to(xd.device)
    nbytes = lib().ccq_moe_f32_workspace_size(T, k, E, H, I)
    ws = _dev.workspace("moe_f32", nbytes, xd.device)
    sd = _shared_rows(shared, T, H, xd.device) if shared is not None else None
    call("ccq_moe_f32_ffn", xd.data_ptr(), ids.data_ptr(), wts.data_ptr(), tab[0].data_ptr(), tab[1].data_ptr(),
         tab[2].data_ptr(), sd.data_ptr() if sd is not None else None, float(np.float32(shared_gate)),
         out.data_ptr(), 0, T, k, E, H, I, ws.data_ptr(), nbytes, _dev.stream_ptr(xd.device))
    return out


def _shared_rows(shared, T: int, H: int, device) -> torch.Tensor:
    sd = _dev.to_device(shared, torch.float32).contiguous()
    if tuple(sd.shape) != (T, H):
        raise ValueError(f"shared expert output must be [{T}, {H}], got {tuple(sd.shape)}")
    return sd.to(device)


def _experts_in_order(sch: dict) -> list[int]:
    """Distinct experts of a tile_m=1 schedule, in first-appearance order."""
    te = sch["tile_expert"][: sch["num_tiles"]].tolist()
    order, last = [], None
    for e in te:
        if e != last:
            order.append(e)
            last = e
    return order


def shared_expert_add(y, shared_out, gate_value: float) -> None:
    """``y += gate_value * shared_out`` in place (reference ``moe.py:177-179``):
    float32, the product rounded, then the add (``ccq_shared_expert_add``).
    The MoE entry points can do this in their combine epilogue instead
    (``moe_combine(..., shared=)``, ``moe_ffn_w4(..., shared=)``)."""
    g = float(np.float32(gate_value))
    if isinstance(y, torch.Tensor) and y.is_cuda and y.dtype == torch.float32 and y.is_contiguous():
        sd = _dev.to_device(shared_out, torch.float32).contiguous().reshape(y.shape)
        call("ccq_shared_expert_add", y.data_ptr(), sd.data_ptr(), g, y.numel(), _dev.stream_ptr(y.device))
        return
    if isinstance(y, torch.Tensor):
        # other dtypes / layouts: the same float32 arithmetic on a float32 copy
        yf = y.float().contiguous()
        shared_expert_add(yf, shared_out, gate_value)
        y.copy_(yf.reshape(y.shape))
        return
    yd = _dev.to_device(np.asarray(y, np.float32))
    shared_expert_add(yd, shared_out, gate_value)
    np.copyto(y, _dev.to_host(yd).reshape(np.shape(y)))


# ---------------------------------------------------------------------------
# fused quantized expert forward (AWQ int4 experts)
# ---------------------------------------------------------------------------


@dataclass
class W4Experts:
    """All experts of one MoE layer, AWQ int4, resident in HBM in the GPU
    layout (tiled weights + packed scale/zero words, see ``quant.awq``).
    gate/up are ``[hidden -> inter]``, down ``[inter -> hidden]``."""

    w_gate: torch.Tensor
    sz_gate: torch.Tensor
    w_up: torch.Tensor
    sz_up: torch.Tensor
    w_down: torch.Tensor
    sz_down: torch.Tensor
    scale_dtype: torch.dtype
    num_experts: int
    hidden: int
    inter: int
    group_size: int = 128
    # the last expert of the stack is the layer's shared expert (every token
    # takes it with the shared gate as weight); num_experts counts it
    shared_expert: bool = False

    @property
    def routed_experts(self) -> int:
        return self.num_experts - (1 if self.shared_expert else 0)

    @staticmethod
    def from_awq(gate: tuple, up: tuple, down: tuple, group_size: int = 128, shared: tuple | None = None
                 ) -> "W4Experts":
        """Each of ``gate``/``up``/``down`` is ``(qweight [E, K, N/8],
        qzeros [E, K/G, N/8], scales [E, K/G, N])`` in AWQ layout.
        ``shared``: the shared expert as ``(gate, up, down)``, each
        ``(qweight [K, N/8], qzeros [K/G, N/8], scales [K/G, N])``, stored
        after the routed experts."""
        if shared is not None:
            def cat(t, one):
                return tuple(torch.cat([_dev.to_device(a), _dev.to_device(b).unsqueeze(0)]) for a, b in zip(t, one))
            gate, up, down = cat(gate, shared[0]), cat(up, shared[1]), cat(down, shared[2])
        def stack(t, K, N):
            qw, qz, sc = (_dev.to_device(a) for a in t)
            E = qw.shape[0]
            qw = qw.view(torch.int32).reshape(E, K, N // 8)
            qz = qz.view(torch.int32).reshape(E, K // group_size, N // 8)
            if sc.dtype not in (torch.float16, torch.bfloat16):
                sc = sc.to(torch.float16)
            sc = sc.reshape(E, K // group_size, N).contiguous()
            tiled = torch.empty_like(qw)
            words = lib().ccq_awq_sz_words(K, group_size)
            sz = torch.empty((E, N, words), dtype=torch.int32, device=qw.device)
            code = 1 if sc.dtype == torch.float16 else 2
            for e in range(E):
                call("ccq_awq_repack", qw[e].data_ptr(), tiled[e].data_ptr(), K, N, _dev.stream_ptr())
                call("ccq_awq_pack_sz", qz[e].contiguous().data_ptr(), sc[e].data_ptr(), code, sz[e].data_ptr(),
                     K, N, group_size, _dev.stream_ptr())
            return tiled, sz, sc.dtype

        if group_size not in (32, 64, 128):
            raise ValueError(f"AWQ group size {group_size} not in (32, 64, 128)")
        E = _dev.to_device(gate[0]).shape[0]
        sg = _dev.to_device(gate[2])
        hidden = sg.shape[1] * group_size
        inter = sg.shape[2]
        g = stack(gate, hidden, inter)
        u = stack(up, hidden, inter)
        d = stack(down, inter, hidden)
        if not (g[2] == u[2] == d[2]):
            raise ValueError("gate, up and down scales must share one dtype")
        return W4Experts(g[0], g[1], u[0], u[1], d[0], d[1], g[2], num_experts=E, hidden=hidden, inter=inter,
                         group_size=group_size, shared_expert=shared is not None)

    def descriptor(self) -> ccq_w4_experts:
        code = 1 if self.scale_dtype == torch.float16 else 2
        return ccq_w4_experts(self.w_gate.data_ptr(), self.sz_gate.data_ptr(), self.w_up.data_ptr(),
                              self.sz_up.data_ptr(), self.w_down.data_ptr(), self.sz_down.data_ptr(),
                              code, self.num_experts, self.hidden, self.inter, self.group_size)

    @property
    def bytes_per_expert(self) -> int:
        """Bytes of one expert in the AWQ format (int4 weights, 16-bit scales,
        int4 zeros of gate, up and down): the algorithmic traffic of reading
        it once."""
        H, I, G = self.hidden, self.inter, self.group_size
        one = H * I // 2 + (H // G) * I * 2 + (H // G) * I // 2
        down = I * H // 2 + (I // G) * H * 2 + (I // G) * H // 2
        return 2 * one + down

    @property
    def gate_up_bytes_per_expert(self) -> int:
        H, I, G = self.hidden, self.inter, self.group_size
        return 2 * (H * I // 2 + (H // G) * I * 2 + (H // G) * I // 2)


def moe_ffn_w4(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, experts: W4Experts,
               out_dtype: torch.dtype | None = None, *, shared=None, shared_gate: float = 1.0) -> torch.Tensor:
    """Expert FFN + weighted combine for already-routed tokens (one call of
    ``ccq_moe_w4_ffn``: align, gate/up + SiLU, down, combine).  ``shared``
    ([T, H] float32, the shared expert's output): ``shared_gate * shared``
    is added in the combine's epilogue (``ccq_moe_w4_ffn_shared``).  When
    the stack holds the shared expert (``experts.shared_expert``), every
    token takes it as one more slot with weight ``shared_gate``: its FFN
    runs in the same kernels and is added after the routed sum."""
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"activations must be float16 or bfloat16, got {x.dtype}")
    x = x.contiguous()
    T, H = x.shape
    if H != experts.hidden:
        raise ValueError(f"x has {H} features, experts expect {experts.hidden}")
    out_dtype = out_dtype or x.dtype
    y = torch.empty((T, H), dtype=out_dtype, device=x.device)
    ids = _dev.to_device(ids).to(torch.int64)
    weights = _dev.to_device(weights).to(torch.float32)
    if experts.shared_expert:
        if shared is not None:
            raise ValueError("the stack holds the shared expert: pass shared_gate only")
        ids = torch.cat([ids, torch.full((T, 1), experts.routed_experts, dtype=torch.int64, device=ids.device)], 1)
        weights = torch.cat([weights, torch.full((T, 1), float(np.float32(shared_gate)), device=weights.device)], 1)
    ids, weights = ids.contiguous(), weights.contiguous()
    k = ids.shape[1]
    desc = experts.descriptor()
    nbytes = lib().ccq_moe_w4_workspace_size(T, k, desc)
    ws = _dev.workspace("moe_w4", nbytes, x.device)
    if shared is not None:
        sd = _shared_rows(shared, T, H, x.device)
        call("ccq_moe_w4_ffn_shared", x.data_ptr(), _dev.DTYPE_CODE[x.dtype], ids.data_ptr(), weights.data_ptr(),
             sd.data_ptr(), float(np.float32(shared_gate)), y.data_ptr(), _dev.DTYPE_CODE[out_dtype], T, k, desc,
             ws.data_ptr(), nbytes, _dev.stream_ptr(x.device))
        return y
    call("ccq_moe_w4_ffn", x.data_ptr(), _dev.DTYPE_CODE[x.dtype], ids.data_ptr(), weights.data_ptr(),
         y.data_ptr(), _dev.DTYPE_CODE[out_dtype], T, k, desc, ws.data_ptr(), nbytes, _dev.stream_ptr(x.device))
    return y


def moe_forward_w4(x: torch.Tensor, router_logits: torch.Tensor, experts: W4Experts, top_k: int,
                   norm_topk_prob: bool = True, out_dtype: torch.dtype | None = None,
                   out: torch.Tensor | None = None, shared_gate: float = 1.0) -> torch.Tensor:
    """Routed MoE layer on AWQ experts: ``topk_softmax`` routing, expert
    grouping, gate/up + SiLU, down and the weighted combine in one call of
    ``ccq_moe_w4_forward`` (the compute of ``ExpertPipeline.step``, reference
    ``experts/pipeline.py:145-179``, and ``moe_forward``,
    ``models/generic.py:361-378``).  Decode batches are routed inside the
    gate/up kernel.  ``out``: optional [T, H] tensor to write (its dtype
    wins over ``out_dtype``).  A stack with the shared expert
    (``experts.shared_expert``) runs ``ccq_moe_w4_forward_shared``: logits
    over the routed experts, the shared expert's FFN in the same kernels,
    ``shared_gate * shared(x)`` added after the routed sum (reference
    ``pipeline.py:181-190``, ``blocks/moe.py:177-179``)."""
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"activations must be float16 or bfloat16, got {x.dtype}")
    x = x.contiguous()
    T, H = x.shape
    if H != experts.hidden:
        raise ValueError(f"x has {H} features, experts expect {experts.hidden}")
    lg = _dev.to_device(router_logits, torch.float32).contiguous()
    E = experts.routed_experts
    if lg.dim() != 2 or lg.shape[0] != T or lg.shape[1] != E:
        raise ValueError(f"router logits must be [{T}, {E}], got {tuple(lg.shape)}")
    if out is None:
        out = torch.empty((T, H), dtype=out_dtype or x.dtype, device=x.device)
    elif out.shape != (T, H) or not out.is_contiguous() or out.device != x.device:
        raise ValueError(f"out must be a contiguous [{T}, {H}] tensor on {x.device}")
    desc = experts.descriptor()
    mode = _MODE_TOPK_THEN_SOFTMAX if norm_topk_prob else _MODE_SOFTMAX_ALL
    if experts.shared_expert:
        nbytes = lib().ccq_moe_w4_workspace_size(T, top_k + 1, desc)
        ws = _dev.workspace("moe_w4", nbytes, x.device)
        call("ccq_moe_w4_forward_shared", x.data_ptr(), _dev.DTYPE_CODE[x.dtype], lg.data_ptr(), T, top_k, mode,
             float(np.float32(shared_gate)), None, None, out.data_ptr(), _dev.DTYPE_CODE[out.dtype], desc,
             ws.data_ptr(), nbytes, _dev.stream_ptr(x.device))
        return out
    nbytes = lib().ccq_moe_w4_workspace_size(T, top_k, desc)
    ws = _dev.workspace("moe_w4", nbytes, x.device)
    call("ccq_moe_w4_forward", x.data_ptr(), _dev.DTYPE_CODE[x.dtype], lg.data_ptr(), T, top_k, mode, None, None,
         out.data_ptr(), _dev.DTYPE_CODE[out.dtype], desc, ws.data_ptr(), nbytes, _dev.stream_ptr(x.device))
    return out


# ---------------------------------------------------------------------------
# fused quantized expert forward (FP8 e4m3fn experts, 128x128 block scales)
# ---------------------------------------------------------------------------


@dataclass
class Fp8Experts:
    """All experts of one MoE layer in block FP8, resident in HBM in the
    MFMA tile layout (``ccq_fp8_block_repack``).  gate/up ``w [E, I, H]``
    with scales ``[E, I/128, H/128]``; down ``w [E, H, I]`` with scales
    ``[E, H/128, I/128]`` (row = output channel, as checkpoints store them)."""

    w_gate: torch.Tensor
    s_gate: torch.Tensor
    w_up: torch.Tensor
    s_up: torch.Tensor
    w_down: torch.Tensor
    s_down: torch.Tensor
    num_experts: int
    hidden: int
    inter: int

    @staticmethod
    def from_block(gate: tuple, up: tuple, down: tuple) -> "Fp8Experts":
        """Each of ``gate``/``up``/``down`` is ``(w [E, N, K] e4m3fn bytes,
        s [E, N/128, K/128] float32)``."""
        def one(t):
            w = _dev.raw_u8(t[0]).reshape(t[0].shape) if isinstance(t[0], torch.Tensor) else \
                _dev.to_device(np.ascontiguousarray(t[0]).view(np.uint8))
            w = w.view(torch.uint8).contiguous()
            sc = _dev.to_device(t[1], torch.float32).contiguous()
            E, N, K = w.shape
            if N % 128 or K % 128 or tuple(sc.shape) != (E, N // 128, K // 128):
                raise ValueError(f"block FP8 expert weights [E, N, K] = {tuple(w.shape)} with scales "
                                 f"{tuple(sc.shape)}: need N, K multiples of 128 and scales [E, N/128, K/128]")
            tiled = torch.empty_like(w)
            for e in range(E):
                call("ccq_fp8_block_repack", w[e].data_ptr(), tiled[e].data_ptr(), N, K, _dev.stream_ptr())
            return tiled, sc, E, N, K

        wg, sg, E, I, H = one(gate)
        wu, su, E2, I2, H2 = one(up)
        wd, sd, E3, H3, I3 = one(down)
        if not (E == E2 == E3 and I == I2 == I3 and H == H2 == H3):
            raise ValueError("gate/up [E, I, H] and down [E, H, I] shapes disagree")
        return Fp8Experts(wg, sg, wu, su, wd, sd, num_experts=E, hidden=H, inter=I)

    def descriptor(self) -> ccq_fp8_experts:
        return ccq_fp8_experts(self.w_gate.data_ptr(), self.s_gate.data_ptr(), self.w_up.data_ptr(),
                               self.s_up.data_ptr(), self.w_down.data_ptr(), self.s_down.data_ptr(),
                               self.num_experts, self.hidden, self.inter)

    @property
    def bytes_per_expert(self) -> int:
        """Bytes of one expert (fp8 weights + float32 block scales of gate,
        up and down): the algorithmic traffic of reading it once."""
        H, I = self.hidden, self.inter
        return 3 * H * I + 3 * (H // 128) * (I // 128) * 4


def moe_ffn_fp8(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, experts: Fp8Experts,
                out_dtype: torch.dtype | None = None, *, shared=None, shared_gate: float = 1.0) -> torch.Tensor:
    """Expert FFN + weighted combine for already-routed tokens on FP8 block
    experts (one call of ``ccq_moe_fp8_ffn``); ``shared`` as in
    :func:`moe_ffn_w4` (``ccq_moe_fp8_ffn_shared``)."""
    if x.dtype not in _dev.DTYPE_CODE:
        raise ValueError(f"activations must be float32, float16 or bfloat16, got {x.dtype}")
    x = x.contiguous()
    T, H = x.shape
    if H != experts.hidden:
        raise ValueError(f"x has {H} features, experts expect {experts.hidden}")
    k = ids.shape[1]
    out_dtype = out_dtype or x.dtype
    y = torch.empty((T, H), dtype=out_dtype, device=x.device)
    desc = experts.descriptor()
    nbytes = lib().ccq_moe_fp8_workspace_size(T, k, desc)
    ws = _dev.workspace("moe_fp8", nbytes, x.device)
    ids = ids.to(torch.int64).contiguous()
    weights = weights.to(torch.float32).contiguous()
    if shared is not None:
        sd = _shared_rows(shared, T, H, x.device)
        call("ccq_moe_fp8_ffn_shared", x.data_ptr(), _dev.DTYPE_CODE[x.dtype], ids.data_ptr(), weights.data_ptr(),
             sd.data_ptr(), float(np.float32(shared_gate)), y.data_ptr(), _dev.DTYPE_CODE[out_dtype], T, k, desc,
             ws.data_ptr(), nbytes, _dev.stream_ptr(x.device))
        return y
    call("ccq_moe_fp8_ffn", x.data_ptr(), _dev.DTYPE_CODE[x.dtype], ids.data_ptr(), weights.data_ptr(),
         y.data_ptr(), _dev.DTYPE_CODE[out_dtype], T, k, desc, ws.data_ptr(), nbytes, _dev.stream_ptr(x.device))
    return y


def moe_forward_fp8(x: torch.Tensor, router_logits: torch.Tensor, experts: Fp8Experts, top_k: int,
                    norm_topk_prob: bool = True, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Routed MoE layer on block-FP8 experts: ``topk_softmax`` then the fused
    FFN (the compute of ``moe_forward``, reference
    ``models/generic.py:361-378``, with the block-scaled FP8 format)."""
    w, ids = topk_softmax(router_logits, top_k, norm_topk_prob)
    return moe_ffn_fp8(x, ids, w, experts, out_dtype)


# ---------------------------------------------------------------------------
# experts in the reference checkpoint's FP8 format (e4m3 [out, in], one scale
# per output row)
# ---------------------------------------------------------------------------


@dataclass
class Fp8RowExperts:
    """All experts of one MoE layer as the reference's checkpoints store them
    and its ``ExpertReader`` reads them (``experts/reader.py:142-251``):
    e4m3 codes ``[out, in]`` with one scale per output row, used in place by
    ``ccq_moe_fp8row_ffn`` (no re-pack).  gate/up ``w [E, I, H]`` with
    ``s [E, I]``; down ``w [E, H, I]`` with ``s [E, H]``; scales float32."""

    w_gate: torch.Tensor
    s_gate: torch.Tensor
    w_up: torch.Tensor
    s_up: torch.Tensor
    w_down: torch.Tensor
    s_down: torch.Tensor
    num_experts: int
    hidden: int
    inter: int

    @staticmethod
    def from_rows(gate: tuple, up: tuple, down: tuple) -> "Fp8RowExperts":
        """Each of ``gate``/``up``/``down`` is ``(w [E, N, K] e4m3fn bytes
        (uint8 or float8_e4m3fn), s [E, N] or [E, N, 1] (BF16 / F16 / F32,
        widened to float32 exactly as the reference's ``_read_scale``))``."""
        def one(t):
            w = t[0]
            if isinstance(w, torch.Tensor):
                w = w.view(torch.uint8) if w.dtype != torch.uint8 else w
                w = _dev.to_device(w.contiguous())
            else:
                w = _dev.to_device(np.ascontiguousarray(w).view(np.uint8))
            sc = _dev.to_device(t[1], torch.float32)
            if w.dim() != 3:
                raise ValueError(f"FP8 expert weights must be [E, N, K], got {tuple(w.shape)}")
            E, N, K = w.shape
            if sc.dim() == 3 and sc.shape[-1] == 1:
                sc = sc.reshape(E, N)
            if tuple(sc.shape) != (E, N):
                raise ValueError(f"per-row scales of a [E, N, K] = {tuple(w.shape)} weight must be [E, N] or "
                                 f"[E, N, 1], got {tuple(sc.shape)}")
            return w, sc.contiguous(), E, N, K

        wg, sg, E, I, H = one(gate)
        wu, su, E2, I2, H2 = one(up)
        wd, sd, E3, H3, I3 = one(down)
        if not (E == E2 == E3 and I == I2 == I3 and H == H2 == H3):
            raise ValueError("gate/up [E, I, H] and down [E, H, I] shapes disagree")
        if H % 256 or I % 256:
            raise ValueError(f"hidden={H} and inter={I} must be multiples of 256 for the fused FP8 kernels")
        return Fp8RowExperts(wg, sg, wu, su, wd, sd, num_experts=E, hidden=H, inter=I)

    def descriptor(self) -> ccq_fp8row_experts:
        return ccq_fp8row_experts(self.w_gate.data_ptr(), self.s_gate.data_ptr(), self.w_up.data_ptr(),
                                  self.s_up.data_ptr(), self.w_down.data_ptr(), self.s_down.data_ptr(),
                                  self.num_experts, self.hidden, self.inter)

    @property
    def bytes_per_expert(self) -> int:
        """Bytes of one expert in its checkpoint form (e4m3 weights + BF16
        row scales of gate, up and down): the algorithmic traffic of reading
        it once."""
        H, I = self.hidden, self.inter
        return 3 * H * I + (2 * I + H) * 2


def moe_ffn_fp8row(x, ids, weights, experts: Fp8RowExperts, out_dtype: torch.dtype = torch.float32, *,
                   shared=None, shared_gate: float = 1.0) -> torch.Tensor:
    """Expert FFN + weighted combine for already-routed float32 tokens on
    per-row FP8 experts, one call of ``ccq_moe_fp8row_ffn`` -- what the
    reference's ``ExpertPipeline.step`` computes per expert with
    ``reader.get`` + ``expert_ffn`` + the weighted add
    (``experts/pipeline.py:155-179``).  ``shared`` [T, H] float32 is added
    as ``shared_gate * shared`` in the combine (``ccq_moe_fp8row_ffn_shared``)."""
    xd = _dev.to_device(x, torch.float32).contiguous()
    if xd.dim() != 2:
        raise ValueError(f"x must be [T, hidden], got {tuple(xd.shape)}")
    T, H = xd.shape
    if H != experts.hidden:
        raise ValueError(f"x has {H} features, experts expect {experts.hidden}")
    ids = _dev.to_device(ids, torch.int64).contiguous()
    wts = _dev.to_device(weights, torch.float32).contiguous()
    if ids.dim() != 2 or ids.shape[0] != T or tuple(wts.shape) != tuple(ids.shape):
        raise ValueError(f"ids {tuple(ids.shape)} and weights {tuple(wts.shape)} must both be [T={T}, k]")
    k = ids.shape[1]
    y = torch.empty((T, H), dtype=out_dtype, device=xd.device)
    desc = experts.descriptor()
    nbytes = lib().ccq_moe_fp8row_workspace_size(T, k, desc)
    ws = _dev.workspace("moe_fp8row", nbytes, xd.device)
    if shared is not None:
        sd = _shared_rows(shared, T, H, xd.device)
        call("ccq_moe_fp8row_ffn_shared", xd.data_ptr(), ids.data_ptr(), wts.data_ptr(), sd.data_ptr(),
             float(np.float32(shared_gate)), y.data_ptr(), _dev.DTYPE_CODE[out_dtype], T, k, desc, ws.data_ptr(),
             nbytes, _dev.stream_ptr(xd.device))
    else:
        call("ccq_moe_fp8row_ffn", xd.data_ptr(), ids.data_ptr(), wts.data_ptr(), y.data_ptr(),
             _dev.DTYPE_CODE[out_dtype], T, k, desc, ws.data_ptr(), nbytes, _dev.stream_ptr(xd.device))
    return y
