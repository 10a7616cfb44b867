"""Drop-in for reference/moe_ref.py (contract v3 MoE and its dense pieces), on MI355X.

Same names and signatures; GPU tensors only; results bit-identical to the reference.

    bfr                                   moe_ref.py:22-24
    rowquant(x)                           moe_ref.py:27-37
    lin_epilogue(acc, ws, asc)            moe_ref.py:40-42
    int_mm(a8, b8)                        moe_ref.py:48-55
    lin_epilogue_b(acc, ws, asc, bias)    moe_ref.py:164-169
    table_scores, router_from_logits, router, router_b     moe_ref.py:64-97, 203-210
    sigmoid_contract, act_swigluoai, act_silu              moe_ref.py:150-186
    expert_swiglu, expert_block                            moe_ref.py:100-114, 189-200
    moe_forward, moe_forward_b                             moe_ref.py:117-140, 213-230
    int_mm_mx, lin_epilogue_mx, expert_block_mx, moe_forward_mx   moe_ref.py:243-290
    blockquant, int_mm_mx2, expert_block_mx2, moe_forward_mx2     moe_ref.py:299-352
"""
from __future__ import annotations

import contextlib
import ctypes
import threading

import torch

from . import _lib as L
from . import ops

BF = torch.bfloat16
F32 = torch.float32
INT8_MIN_ROWS = 17   # API compatibility only: the kernels take any row count
# The fused layers read the activation's gate part from a per-device table of all bf16 gate values
# (ops.act_table); False evaluates it step by step in the epilogues (the same bits, slower).
USE_ACT_TABLE = True


def _act_tab(dev, act: int):
    return ops.act_table(dev, act).data_ptr() if USE_ACT_TABLE else None


def bfr(x: torch.Tensor) -> torch.Tensor:
    """fl32 -> bf16 -> fl32 (torch's own RNE conversion, which the kernels reproduce)."""
    return x.to(BF).to(F32)


def rowquant(x: torch.Tensor):
    """asc = max(|x|, 1e-8) / 127 (a true division), q = clamp(rint(x / asc), +-127) per row.
    x [..., K] -> (q int8 [..., K], asc f32 [...])."""
    return ops.rowquant(x)


def lin_epilogue(acc: torch.Tensor, ws: torch.Tensor, asc: torch.Tensor) -> torch.Tensor:
    """y8 = bf16((fl32(acc) * ws[n]) * asc[m]), returned in binary32."""
    return ops.epilogue(acc, L.EPI_V21, L.LSK_BF16_AS_F32, asc=asc, ws=ws)


def lin_epilogue_b(acc: torch.Tensor, ws: torch.Tensor, asc: torch.Tensor, bias=None) -> torch.Tensor:
    """bfr(bfr(fl32(acc) * ws * asc) + b)."""
    return ops.epilogue(acc, L.EPI_V21, L.LSK_BF16_AS_F32, asc=asc, ws=ws, bias=bias)


def int_mm(a8: torch.Tensor, b8: torch.Tensor) -> torch.Tensor:
    """int8 [M, K] x int8 [K, N] -> int32 [M, N], exact, any M >= 0."""
    return ops.gemm(a8, ops.weight_nk(b8), L.EPI_RAW, L.LSK_I32)


def linear(q: torch.Tensor, asc: torch.Tensor, b8: torch.Tensor, ws: torch.Tensor, bias=None) -> torch.Tensor:
    """lin_epilogue_b(int_mm(q, b8), ws, asc, bias) in one launch (the fused form)."""
    return ops.gemm(q, ops.weight_nk(b8), L.EPI_V21, L.LSK_BF16_AS_F32, asc=asc, ws=ws, bias=bias)


# ============================================================================ router (moe_ref.py:58-97, 203-210)
BHI, TAB_N, TAB_W = 26, 13, 15
ROUTER_C = float(2.0 ** BHI / 0.6931471805599453)   # rounded once to binary32 by the kernels
SWIGLU_ALPHA = torch.tensor(1.702, dtype=F32)
SWIGLU_LIMIT = 7.0


def table_scores(dgap: torch.Tensor, tab: torch.Tensor) -> torch.Tensor:
    """Integer router scores of the gaps dgap >= 0: the attention rule's table exponential."""
    return ops.table_scores(dgap, tab)


def router_from_logits(g: torch.Tensor, k: int, renormalize: bool, tab: torch.Tensor, win: int = 0):
    """Top-k by table score (ties to the lower expert index) and w = bf16(s / S).
    Returns (idx int64 [T, k] by rank, w bf16 [T, k], g bf16 [T, E])."""
    idx, w = ops.router_topk(g, k, renormalize, tab)
    return idx, w, g.to(BF)


def router(x: torch.Tensor, gate_w8: torch.Tensor, gate_ws: torch.Tensor, k: int, renormalize: bool,
           tab: torch.Tensor, win: int = 0):
    """rowquant -> exact GEMM with the [H, E] gate -> v2.1 epilogue -> router_from_logits."""
    q, asc = rowquant(x)
    g = linear(q, asc, gate_w8, gate_ws)
    return router_from_logits(g, k, renormalize, tab, win)


def router_b(x, gate_w8, gate_ws, k, renormalize, tab, win, gate_bias=None):
    """The router with an optional bias on the gate logits (a second bf16 rounding)."""
    if gate_bias is None:
        return router(x, gate_w8, gate_ws, k, renormalize, tab, win)
    q, asc = rowquant(x)
    g = linear(q, asc, gate_w8, gate_ws, gate_bias).to(BF)
    return router_from_logits(g, k, renormalize, tab, win)


# ============================================================================ activations (moe_ref.py:150-186)
def sigmoid_contract(x: torch.Tensor) -> torch.Tensor:
    """Steps (1)-(9) of the invariant SiLU: the table sigmoid, binary32 in and out."""
    return ops.act(x, None, ops.OP_SIGMOID)


def act_swigluoai(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """GPT-OSS clamped SwiGLU with the alpha-scaled table sigmoid; bf16 values in binary32."""
    return ops.act(gate, up, ops.OP_ACT_SWIGLUOAI)


def act_silu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """bfr(silu_table(g) * u)."""
    return ops.act(gate, up, ops.OP_ACT_SILU)


def _act_code(fn) -> int:
    name = getattr(fn, "__name__", "")
    if fn is act_silu or name == "act_silu":
        return L.LSK_ACT_SILU
    if fn is act_swigluoai or name == "act_swigluoai":
        return L.LSK_ACT_SWIGLUOAI
    raise NotImplementedError("the fused MoE layer runs the contract activations act_silu / act_swigluoai; "
                              "got %r" % (fn,))


# ============================================================================ expert blocks (moe_ref.py:100-114, 189-200)
def _fwht(v, blk, scale):
    return ops.fwht_blocks(v.to(F32), blk, scale)


def expert_swiglu(x_rows, w13_8, ws13, w2_8, ws2, silu_fn, rot: bool = False):
    """The v2.5 SwiGLU block on one expert's rows (w13_8 [H, 2I], w2_8 [I, H] column-major)."""
    xin = _fwht(x_rows, 256, 1.0 / 16.0) if rot else x_rows
    q, asc = rowquant(xin)
    y = linear(q, asc, w13_8, ws13)
    I = y.shape[-1] // 2
    h = silu_fn(y[:, :I], y[:, I:])
    hin = _fwht(h, 256, 1.0 / 16.0) if rot else h
    q2, asc2 = rowquant(hin)
    return linear(q2, asc2, w2_8, ws2)


def expert_block(x_rows, w13_8, ws13, w2_8, ws2, act, b13=None, b2=None, rot_blk: int = 256):
    """The expert block with biases and a parametrised R1 / R4 block (0 = no rotation)."""
    def rot(v):
        if not rot_blk:
            return v
        return _fwht(v, rot_blk, 1.0 / (rot_blk ** 0.5))
    q, asc = rowquant(rot(x_rows))
    y = linear(q, asc, w13_8, ws13, b13)
    I = y.shape[-1] // 2
    h = act(y[:, :I], y[:, I:])
    q2, asc2 = rowquant(rot(h))
    return linear(q2, asc2, w2_8, ws2, b2)


# ============================================================================ the fused layer (moe_ref.py:117-140, 213-230)
# ExpertTables keep a row-pair copy of every int8 expert weight (one more copy of the weights in
# HBM; the ping-pong expert tiles read it faster).  False: the tables read the weights alone.
ROW_PAIRS = True


class ExpertTables:
    """Device address tables of the experts' int8 weights, scales and biases, as the fused
    layer reads them.  experts[e] = (w13col [H, 2I], ws13 [2I], w2col [I, H], ws2 [H][, b13, b2]),
    each w*col the transpose view of a row-major [N, K] int8 matrix (else it is copied once)."""

    def __init__(self, experts):
        if not experts:
            raise ValueError("no experts")
        ex0 = experts[0]
        L.require_cuda(ex0[0], what="experts")
        self.device = ex0[0].device
        self.E = len(experts)
        self.H = int(ex0[0].shape[0])
        self.I = int(ex0[0].shape[1]) // 2
        keep, pairs = [], []
        w13, ws13, w2, ws2, b13, b2 = [], [], [], [], [], []
        for ex in experts:
            W13 = ops.weight_nk(ex[0])
            W2 = ops.weight_nk(ex[2])
            if W13.dtype != torch.int8 or W2.dtype != torch.int8:
                raise TypeError("expert weights must be int8")
            if tuple(W13.shape) != (2 * self.I, self.H) or tuple(W2.shape) != (self.H, self.I):
                raise ValueError("expert shapes differ: %s / %s" % (tuple(W13.shape), tuple(W2.shape)))
            s13 = ex[1].to(F32).contiguous()
            s2 = ex[3].to(F32).contiguous()
            c13 = ex[4].to(F32).contiguous() if len(ex) > 4 and ex[4] is not None else None
            c2 = ex[5].to(F32).contiguous() if len(ex) > 5 and ex[5] is not None else None
            keep += [W13, W2, s13, s2, c13, c2]
            pairs += [(ex[1], s13), (ex[3], s2)] + ([(ex[4], c13)] if c13 is not None else []) + \
                     ([(ex[5], c2)] if c2 is not None else [])
            w13.append(W13)
            w2.append(W2)
            ws13.append(s13.data_ptr())
            ws2.append(s2.data_ptr())
            b13.append(c13.data_ptr() if c13 is not None else 0)
            b2.append(c2.data_ptr() if c2 is not None else 0)
        ld13 = {t.stride(0) for t in w13}
        ld2 = {t.stride(0) for t in w2}
        if len(ld13) != 1 or ld13.pop() % 16 or any(t.stride(0) != w13[0].stride(0) for t in w13):
            w13 = [t.contiguous() for t in w13]
            keep += w13
        if len(ld2) != 1 or w2[0].stride(0) % 16:
            w2 = [t.contiguous() for t in w2]
            keep += w2
        self.ldw13 = int(w13[0].stride(0))
        self.ldw2 = int(w2[0].stride(0))
        dev = self.device

        def table(vals):
            return torch.tensor(vals, dtype=torch.int64).to(dev)
        self.w13 = table([t.data_ptr() for t in w13])
        self.w2 = table([t.data_ptr() for t in w2])
        self.ws13 = table(ws13)
        self.ws2 = table(ws2)
        self.b13 = table(b13) if any(b13) else None
        self.b2 = table(b2) if any(b2) else None
        # the weights' row-pair copies, which the ping-pong expert tiles read in whole 128-byte
        # lines (the decode GEMVs and the other tiles read the weights above): made by pair_ptrs()
        # on the first call that reads them, held by each weight tensor (ops.row_pair_copy)
        self.w13_pairs = self.w2_pairs = None
        self._w13, self._w2 = w13, w2
        self._keep = keep
        pairs += [(ex[0], t) for ex, t in zip(experts, w13)] + [(ex[2], t) for ex, t in zip(experts, w2)]
        # an in-place update of an int8 weight makes its row-pair copy stale as well
        self._weights = [(ex[0], ex[0]._version) for ex in experts] + [(ex[2], ex[2]._version) for ex in experts]
        self._derived = _derived(pairs)

    def pair_ptrs(self, T, k, rot_blk, select):
        """(w13_pair_ptrs, w2_pair_ptrs) for a layer call of T tokens, top-k: the tables of the experts'
        row-pair copies when that call reads them (lsk_moe_reads_row_pairs), else (None, None)."""
        if not L.load().lsk_moe_reads_row_pairs(int(T), int(k), self.E, self.H, self.I, int(rot_blk), int(select)):
            return None, None
        return self.make_pairs()

    def make_pairs(self):
        """(w13_pair_ptrs, w2_pair_ptrs): the row-pair copy tables, made on first use; (None, None)
        with ROW_PAIRS off, widths not multiples of 16, or while a graph is being captured."""
        if not ROW_PAIRS or self.H % 16 or self.I % 16:
            return None, None
        if self.w13_pairs is None:
            p13 = [ops.row_pair_copy(t) for t in self._w13]
            p2 = [ops.row_pair_copy(t) for t in self._w2]
            if any(t is None for t in p13 + p2):
                return None, None              # (being captured into a graph: the weights themselves)
            dev = self.device
            self._pairs_keep = p13 + p2
            self.w13_pairs = torch.tensor([t.data_ptr() for t in p13], dtype=torch.int64).to(dev)
            self.w2_pairs = torch.tensor([t.data_ptr() for t in p2], dtype=torch.int64).to(dev)
        return self.w13_pairs, self.w2_pairs


def _derived(pairs):
    """(source, version) of every source tensor a table reads through a copy: an in-place update of
    such a source makes the table stale; sources used in place need no check."""
    return [(src, src._version) for src, used in pairs if used.data_ptr() != src.data_ptr()]


# Tables of the experts lists the layers have seen, keyed by the list and its per-expert tuples.  A
# table holds device address tables (a few KB) and references to the list's tensors; the large
# derived data, the int8 weights' row-pair copies, is held by the weight tensors themselves
# (ops.row_pair_copy), so a table rebuilt after eviction re-packs nothing.  TABLES_MAX bounds how
# many lists keep their tensors referenced here (more than the MoE layers of the largest model
# served: Qwen3-30B-A3B has 48).
_TABLES = {}
TABLES_MAX = 256


def _cached(kind, experts, build):
    """The cached tables of an experts list: keyed by the list and its per-expert tuples (cheap: one
    id per expert), valid while every source read through a copy keeps its version."""
    key = (kind, id(experts), tuple(map(id, experts)))
    hit = _TABLES.get(key)
    if hit is not None and hit._src is experts and all(t._version == v for t, v in hit._derived) \
            and all(t._version == v for t, v in getattr(hit, "_weights", ())):
        _TABLES[key] = _TABLES.pop(key)       # most recently used last
        return hit
    _TABLES.pop(key, None)
    while len(_TABLES) >= TABLES_MAX:
        _TABLES.pop(next(iter(_TABLES)))
    hit = _TABLES[key] = build(experts)
    hit._src = experts
    return hit


def expert_tables(experts) -> ExpertTables:
    """Cached ExpertTables for an experts list."""
    if isinstance(experts, ExpertTables):
        return experts
    return _cached("int8", experts, ExpertTables)


def _route_fields(x, route):
    """Routing inside the layer: route = (logits [T, E], k, renormalize, tab).  Returns (idx, w, the
    lsk_moe_args fields, the tensors the fields point at), idx / w the outputs the layer fills --
    the same values as router_from_logits(logits, k, renormalize, tab)."""
    g, k, renormalize, tab = route
    L.require_cuda(g, tab, what="moe_forward")
    T = x.shape[0]
    if g.dim() != 2 or g.shape[0] != T:
        raise ValueError("moe_forward: logits must be [T, E] with T = %d rows" % T)
    if g.dtype == torch.bfloat16:
        gd, code = g.contiguous(), L.LSK_BF16
    else:
        gd, code = g.to(torch.float32).contiguous(), L.LSK_F32
    tb = ops.tab_i32(tab)
    idx = torch.empty((T, int(k)), dtype=torch.int64, device=x.device)
    w = torch.empty((T, int(k)), dtype=BF, device=x.device)
    fields = dict(logits=gd.data_ptr(), logits_dtype=code, renormalize=1 if renormalize else 0, ld_logits=gd.shape[1],
                  router_tab=tb.data_ptr(), idx_out=idx.data_ptr(), w_out=w.data_ptr())
    return idx, w, fields, (gd, tb)


_CHOICE = threading.local()


@contextlib.contextmanager
def kernel_choice(moe=None, mx=None):
    """The MoE layers called inside run with this kernel choice, passed per call
    (lsk_moe_args.select / mx_select; no reference counterpart, the same bits either way): moe as
    lsk_moe_select's variant (-1 by size, 0 register-staged tile, 1 ping-pong tile, 2 GEMV, 3 the
    four-wave tile, 4 128-byte K stages, 5 the persistent 256x256 tile, 6 the 256x256 tile one per
    block, 7 the skinny grouped GEMM), mx as lsk_moe_mx_select's (0, 1, 2, 3); None keeps the calling
    thread's setting.  Scoped to this Python thread and the with-block."""
    if moe is not None and not -1 <= moe <= 7:
        raise ValueError("kernel_choice: moe=%r not in [-1, 7]" % (moe,))
    if mx is not None and not 0 <= mx <= 3:
        raise ValueError("kernel_choice: mx=%r not in [0, 3]" % (mx,))
    prev = getattr(_CHOICE, "v", (0, 0))
    _CHOICE.v = (0 if moe is None else moe + 2, 0 if mx is None else mx + 1)
    try:
        yield
    finally:
        _CHOICE.v = prev


def _choice_fields():
    sel, mxsel = getattr(_CHOICE, "v", (0, 0))
    return {"select": sel, "mx_select": mxsel}


def _moe_layer(x, idx, w, tables: ExpertTables, act: int, rot_blk: int, shared_out=None, route=None):
    """The layer on given routing (idx, w), or with route = (logits, k, renormalize, tab) on the
    routing it computes itself; returns y, or (y, idx, w) with route."""
    fields, keep = {}, None
    if route is not None:
        idx, w, fields, keep = _route_fields(x, route)
    L.require_cuda(x, idx, w, what="moe_forward")
    if x.dtype != BF:
        raise TypeError("moe_forward: x must be bf16 [T, H] (got %s)" % x.dtype)
    x = x.contiguous()
    T, H = x.shape
    k = int(idx.shape[1])
    if H != tables.H:
        raise ValueError("moe_forward: x width %d != expert H %d" % (H, tables.H))
    idx = idx.to(torch.int64).contiguous()
    w = w.to(BF).contiguous()
    y = torch.empty((T, H), dtype=BF, device=x.device)
    if T == 0:
        return y if route is None else (y, idx, w)
    nbytes = L.load().lsk_moe_workspace(T, k, tables.E, H, tables.I, rot_blk, 0)
    work = torch.empty((nbytes,), dtype=torch.uint8, device=x.device)
    sh = None if shared_out is None else shared_out.to(F32).contiguous()
    choice = _choice_fields()
    p13, p2 = tables.pair_ptrs(T, k, rot_blk, choice["select"])
    a = L.MoeArgs(T=T, H=H, I=tables.I, E=tables.E, k=k, act=act, x=x.data_ptr(), idx=idx.data_ptr(),
                  w=w.data_ptr(), w13_ptrs=tables.w13.data_ptr(), ldw13=tables.ldw13,
                  ws13_ptrs=tables.ws13.data_ptr(),
                  b13_ptrs=tables.b13.data_ptr() if tables.b13 is not None else None,
                  w2_ptrs=tables.w2.data_ptr(), ldw2=tables.ldw2, ws2_ptrs=tables.ws2.data_ptr(),
                  b2_ptrs=tables.b2.data_ptr() if tables.b2 is not None else None,
                  frac=ops.frac_i32(x.device).data_ptr(), act_tab=_act_tab(x.device, act), rot_blk=int(rot_blk),
                  rot_scale=(1.0 / (rot_blk ** 0.5)) if rot_blk else 0.0,
                  shared=sh.data_ptr() if sh is not None else None, y=y.data_ptr(),
                  workspace=work.data_ptr(), workspace_bytes=nbytes,
                  w13_pair_ptrs=p13.data_ptr() if p13 is not None else None,
                  w2_pair_ptrs=p2.data_ptr() if p2 is not None else None,
                  **fields, **choice)
    L.call("lsk_moe_forward", ctypes.addressof(a), L.stream_of(x))
    del keep
    return y if route is None else (y, idx, w)


def moe_forward(x: torch.Tensor, gate, experts, k: int, renormalize: bool, tab: torch.Tensor, win: int, silu_fn,
                shared=None, routing=None, rot: bool = False, logits=None):
    """x bf16 [T, H] -> (y bf16 [T, H], idx, w).  routing=(idx, w) injects a routing; the
    declared router runs otherwise.  experts: the reference's list, or an ExpertTables.
    logits (no reference counterpart as one call): router logits [T, E] whose routing the layer
    computes itself -- the same results as routing=router_from_logits(logits, k, renormalize,
    tab)[:2], in fewer launches."""
    if logits is not None:
        sh = shared(x) if shared is not None else None
        return _moe_layer(x, None, None, expert_tables(experts), _act_code(silu_fn), 256 if rot else 0, sh,
                          route=(logits, k, renormalize, tab))
    if routing is None:
        idx, w, _ = router(x, gate[0], gate[1], k, renormalize, tab, win)
    else:
        idx, w = routing[0].to(torch.int64), routing[1].to(BF)
    tables = expert_tables(experts)
    sh = shared(x) if shared is not None else None
    y = _moe_layer(x, idx, w, tables, _act_code(silu_fn), 256 if rot else 0, sh)
    return y, idx, w


def moe_forward_b(x, gate, experts, k, renormalize, tab, win, act, rot_blk=256, routing=None):
    """moe_forward for the GPT-OSS addendum: biased gate and experts, act_silu or
    act_swigluoai, rot_blk the R1 / R4 block (0 = none)."""
    if routing is None:
        idx, w, _ = router_b(x, gate[0], gate[1], k, renormalize, tab, win, gate[2] if len(gate) > 2 else None)
    else:
        idx, w = routing[0].to(torch.int64), routing[1].to(BF)
    y = _moe_layer(x, idx, w, expert_tables(experts), _act_code(act), int(rot_blk or 0))
    return y, idx, w


# ============================================================================ the MXFP4 operand (moe_ref.py:233-290)
MX_BLOCK = 32


def int_mm_mx(a8: torch.Tensor, m2: torch.Tensor, kexp: torch.Tensor) -> torch.Tensor:
    """a8 int8 [T, K]; m2 int8 [N, K] doubled mantissas; kexp [N, K/32] E8M0 -> binary32 [T, N]:
    per 32-block s (exact) then acc = fl32(acc + s * 2^(kexp - 128)) in ascending block order."""
    return ops.gemm_mx(a8, m2, kexp, 0)


def lin_epilogue_mx(acc: torch.Tensor, asc: torch.Tensor, bias=None) -> torch.Tensor:
    """bfr(acc * asc[m]), then bfr(y + b)."""
    return ops.mx_epilogue(acc, asc, bias)


def expert_block_mx(x_rows, w13, w2, act, b13=None, b2=None):
    """w13 = (m2 [2I, H], kexp [2I, H/32]); w2 = (m2 [H, I], kexp [H, I/32]).  No rotation."""
    q, asc = rowquant(x_rows)
    y = ops.gemm_mx(q, w13[0], w13[1], 0, asc=asc, bias=b13, epilogue=1)
    I = y.shape[-1] // 2
    h = act(y[:, :I], y[:, I:])
    q2, asc2 = rowquant(h)
    return ops.gemm_mx(q2, w2[0], w2[1], 0, asc=asc2, bias=b2, epilogue=1)


class ExpertTablesMX:
    """Device address tables of MXFP4 experts as the fused layer reads them: packed E2M1 codes
    [N, K/2] and E8M0 bytes [N, K/32] per projection.  experts[e] = ((m2_13, kexp_13),
    (m2_2, kexp_2), b13 | None, b2 | None) as moe_ref passes them (the m2 are packed once,
    losslessly), or ((packed_13, scale_13), (packed_2, scale_2), ...) with packed=True."""

    def __init__(self, experts, packed: bool = False):
        if not experts:
            raise ValueError("no experts")
        first = experts[0][0][0]
        L.require_cuda(first, what="experts")
        self.device = first.device
        self.E = len(experts)
        keep, pairs = [], []
        p13, s13, p2, s2, b13, b2 = [], [], [], [], [], []
        kw = []
        for ex in experts:
            (m13, k13), (m2_, k2_) = ex[0], ex[1]
            c13 = m13.to(torch.uint8).contiguous() if packed else ops.pack_m2(m13)
            c2 = m2_.to(torch.uint8).contiguous() if packed else ops.pack_m2(m2_)
            e13 = k13.to(torch.uint8).contiguous()
            e2 = k2_.to(torch.uint8).contiguous()
            bb13 = ex[2].to(F32).contiguous() if len(ex) > 2 and ex[2] is not None else None
            bb2 = ex[3].to(F32).contiguous() if len(ex) > 3 and ex[3] is not None else None
            keep += [c13, c2, e13, e2, bb13, bb2]
            p13.append(c13.data_ptr())
            p2.append(c2.data_ptr())
            s13.append(e13.data_ptr())
            s2.append(e2.data_ptr())
            b13.append(bb13.data_ptr() if bb13 is not None else 0)
            b2.append(bb2.data_ptr() if bb2 is not None else 0)
            pairs += [(m13, c13), (m2_, c2), (k13, e13), (k2_, e2)] + \
                     ([(ex[2], bb13)] if bb13 is not None else []) + ([(ex[3], bb2)] if bb2 is not None else [])
            kw.append(torch.stack([e13.min(), e13.max(), e2.min(), e2.max()]).to(torch.int32))
        two_i, hh = keep[0].shape
        self.I = int(two_i) // 2
        self.H = int(hh) * 2
        self.ldw13, self.ldw2 = int(keep[0].stride(0)), int(keep[1].stride(0))
        self.lds13, self.lds2 = int(keep[2].stride(0)), int(keep[3].stride(0))
        # E8M0 bounds over all experts (w13 min / max, w2 min / max), one host synchronisation: the
        # multiply-then-add update once an exponent reaches 240; block-scaled activations use them all
        kr = torch.stack(kw).cpu()
        self.kw_bounds = (int(kr[:, 0].min()), int(kr[:, 1].max()), int(kr[:, 2].min()), int(kr[:, 3].max()))
        self.mx_safe = 1 if max(self.kw_bounds[1], self.kw_bounds[3]) >= 240 else 0
        dev = self.device

        def table(vals):
            return torch.tensor(vals, dtype=torch.int64).to(dev)
        self.w13, self.w2, self.ws13, self.ws2 = table(p13), table(p2), table(s13), table(s2)
        self.b13 = table(b13) if any(b13) else None
        self.b2 = table(b2) if any(b2) else None
        self._keep = keep
        self._derived = _derived(pairs)
        # the codes' skinny-layout copies (lsk_mx_skinny_pack), which the skinny grouped MX GEMM
        # reads a kilobyte per wave load: made by make_skinny() on the first call that reads them,
        # remade when a code tensor changes in place
        self._codes = [keep[i] for i in range(0, len(keep), 6)] + [keep[i] for i in range(1, len(keep), 6)]
        self._skinny = [None, None]

    def skinny_ptrs(self, T, k, select, mx_select):
        """(w13_pair_ptrs, w2_pair_ptrs) for an MXFP4 layer call (per-row scales) of T tokens, top-k:
        the tables of the skinny-layout code copies when that call reads them
        (lsk_moe_mx_reads_skinny), else (None, None); (None, None) while a graph is being captured
        (the graph then runs the kernels that read the codes themselves)."""
        if not L.load().lsk_moe_mx_reads_skinny(int(T), int(k), self.E, self.H, self.I, self.lds13, self.lds2,
                                                int(select), int(mx_select)):
            return None, None
        t13, t2 = self.make_skinny(0), self.make_skinny(1)
        return (t13, t2) if t13 is not None and t2 is not None else (None, None)

    def make_skinny(self, j):
        """The device table of projection j's (0: w13 [2I, H/2], 1: w2 [H, I/2]) skinny-layout code
        copies, made on first use and remade after an in-place update of those codes; None where its
        K is not a multiple of 32 or while a graph is being captured before they exist."""
        rows, K = (2 * self.I, self.H) if j == 0 else (self.H, self.I)
        if K % 32:
            return None
        codes = self._codes[j * self.E:(j + 1) * self.E]
        vers = [c._version for c in codes]
        hit = self._skinny[j]
        if hit is not None and hit[0] == vers:
            return hit[2]
        if torch.cuda.is_current_stream_capturing():
            return None
        self._skinny[j] = None                  # stale: freed before the new copies are made
        lib = L.load()
        copies = []
        for c in codes:
            out = torch.empty((lib.lsk_mx_skinny_bytes(rows, K),), dtype=torch.uint8, device=self.device)
            L.call("lsk_mx_skinny_pack", L.ptr(c), int(c.stride(0)), rows, K, L.ptr(out), L.stream_of(out))
            copies.append(out)
        table = torch.tensor([t.data_ptr() for t in copies], dtype=torch.int64).to(self.device)
        self._skinny[j] = (vers, copies, table)
        return table


def expert_tables_mx(experts) -> ExpertTablesMX:
    if isinstance(experts, ExpertTablesMX):
        return experts
    return _cached("mx", experts, ExpertTablesMX)


# ============================================================================ one grouped expert linear
def _grouped_common(tables, which, a, asc, offs, what):
    if which not in ("w13", "w2"):
        raise ValueError("%s: which must be 'w13' or 'w2'" % what)
    L.require_cuda(a, asc, offs, what=what)
    if offs.dtype != torch.int32 or offs.dim() != 1 or offs.numel() != tables.E + 1:
        raise ValueError("%s: offs must be int32 [E + 1] = [%d]" % (what, tables.E + 1))
    R = a.shape[0]
    N = 2 * tables.I if which == "w13" else tables.H
    out = torch.empty((R, N), dtype=BF, device=a.device)
    nbytes = L.load().lsk_grouped_gemm_workspace(R, tables.E)
    work = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=a.device)
    return R, N, out, work, nbytes


def grouped_linear(tables, which: str, a8, asc, offs):
    """One projection of every expert over rows already sorted by expert (expert e owns rows
    offs[e] .. offs[e + 1] - 1): per expert lin_epilogue(_b)(int_mm(a8[rows], w_col_e), ws_e, asc[rows]
    [, b_e]) -- the per-expert linears of expert_block (moe_ref.py:189-200, :40-55, :164-169) as one
    grouped launch, bf16 out [R, N].  tables: ExpertTables; which: 'w13' (N = 2I, K = H) or 'w2'
    (N = H, K = I); a8 int8 [R, K]; asc f32 [R]; offs int32 [E + 1] on the device."""
    tables = expert_tables(tables)
    R, N, out, work, nbytes = _grouped_common(tables, which, a8, asc, offs, "grouped_linear")
    w, ws, b = (tables.w13, tables.ws13, tables.b13) if which == "w13" else (tables.w2, tables.ws2, tables.b2)
    ldw = tables.ldw13 if which == "w13" else tables.ldw2
    a8 = a8 if a8.stride(-1) == 1 else a8.contiguous()
    asc = asc.to(F32).contiguous()
    # the ping-pong tiles, which read the row-pair copies, run once experts average 16 rows
    wp = tables.make_pairs()[0 if which == "w13" else 1] if R >= 16 * tables.E else None
    L.call("lsk_grouped_gemm_w8a8_pairs", L.ptr(a8), a8.stride(0) if R > 1 else a8.shape[1], L.ptr(asc),
           L.ptr(offs), tables.E, R, L.ptr(w), ldw, L.ptr(wp), L.ptr(ws), L.ptr(b), N, a8.shape[1], L.ptr(out),
           L.ptr(work), nbytes, L.stream_of(a8))
    return out


def grouped_linear_mx(tables, which: str, a8, asc, offs):
    """The MXFP4 form (moe_ref.py:243-261 per expert, as expert_block_mx :264-271 runs them):
    lin_epilogue_mx(int_mm_mx(a8[rows], m2_e, kexp_e), asc[rows][, b_e]) over expert-sorted rows.
    a8: the int8 row values [R, K] (int8, or held as bf16 as the MX kernels read them)."""
    tables = expert_tables_mx(tables)
    R, N, out, work, nbytes = _grouped_common(tables, which, a8, asc, offs, "grouped_linear_mx")
    ab = a8 if a8.dtype == BF else a8.to(BF)        # int8 values are exact in bf16
    ab = ab if ab.stride(-1) == 1 else ab.contiguous()
    w, kx, b = (tables.w13, tables.ws13, tables.b13) if which == "w13" else (tables.w2, tables.ws2, tables.b2)
    ldw, lds = (tables.ldw13, tables.lds13) if which == "w13" else (tables.ldw2, tables.lds2)
    asc = asc.to(F32).contiguous()
    # experts averaging few rows: the skinny grouped MX GEMM on the codes' skinny-layout copies
    wsk = None
    if L.load().lsk_grouped_mx_reads_skinny(R, tables.E, ab.shape[1], lds):
        wsk = tables.make_skinny(0 if which == "w13" else 1)
    L.call("lsk_grouped_gemm_mx_skinny", L.ptr(ab), ab.stride(0) if R > 1 else ab.shape[1], L.ptr(asc),
           L.ptr(offs), tables.E, R, L.ptr(w), ldw, L.ptr(wsk), L.ptr(kx), lds, L.ptr(b), N, ab.shape[1],
           tables.mx_safe, L.ptr(out), L.ptr(work), nbytes, L.stream_of(ab))
    return out


def _moe_layer_mx(x, idx, w, t: ExpertTablesMX, act: int, wfmt: int = 1, route=None):
    what = "moe_forward_mx2" if wfmt == 2 else "moe_forward_mx"
    fields, keep = {}, None
    if route is not None:
        idx, w, fields, keep = _route_fields(x, route)
    L.require_cuda(x, idx, w, what=what)
    if x.dtype != BF:
        raise TypeError("%s: x must be bf16 [T, H] (got %s)" % (what, x.dtype))
    x = x.contiguous()
    T, H = x.shape
    k = int(idx.shape[1])
    if H != t.H:
        raise ValueError("moe_forward_mx: x width %d != expert H %d" % (H, t.H))
    idx = idx.to(torch.int64).contiguous()
    w = w.to(BF).contiguous()
    y = torch.empty((T, H), dtype=BF, device=x.device)
    if T == 0:
        return y if route is None else (y, idx, w)
    nbytes = L.load().lsk_moe_workspace(T, k, t.E, H, t.I, 0, wfmt)
    work = torch.empty((nbytes,), dtype=torch.uint8, device=x.device)
    kb = t.kw_bounds
    choice = _choice_fields()
    s13, s2 = t.skinny_ptrs(T, k, choice["select"], choice["mx_select"])
    a = L.MoeArgs(T=T, H=H, I=t.I, E=t.E, k=k, act=act, wfmt=wfmt, mx_safe=t.mx_safe, lds13=t.lds13, lds2=t.lds2,
                  kw13_min=kb[0], kw13_max=kb[1], kw2_min=kb[2], kw2_max=kb[3],
                  x=x.data_ptr(), idx=idx.data_ptr(), w=w.data_ptr(), w13_ptrs=t.w13.data_ptr(), ldw13=t.ldw13,
                  ws13_ptrs=t.ws13.data_ptr(), b13_ptrs=t.b13.data_ptr() if t.b13 is not None else None,
                  w2_ptrs=t.w2.data_ptr(), ldw2=t.ldw2, ws2_ptrs=t.ws2.data_ptr(),
                  b2_ptrs=t.b2.data_ptr() if t.b2 is not None else None, frac=ops.frac_i32(x.device).data_ptr(),
                  act_tab=_act_tab(x.device, act), rot_blk=0, rot_scale=0.0, shared=None, y=y.data_ptr(), workspace=work.data_ptr(),
                  workspace_bytes=nbytes, w13_pair_ptrs=s13.data_ptr() if s13 is not None else None,
                  w2_pair_ptrs=s2.data_ptr() if s2 is not None else None, **fields, **choice)
    L.call("lsk_moe_forward", ctypes.addressof(a), L.stream_of(x))
    del keep
    return y if route is None else (y, idx, w)


def moe_forward_mx(x, gate, experts, k, renormalize, tab, win, act, routing=None, logits=None):
    """experts[e] = ((m2_13, kexp_13), (m2_2, kexp_2), b13 | None, b2 | None), or an
    ExpertTablesMX; gate as moe_forward_b.  Returns (y bf16 [T, H], idx, w).  logits: as
    moe_forward's."""
    if logits is not None:
        return _moe_layer_mx(x, None, None, expert_tables_mx(experts), _act_code(act), route=(logits, k, renormalize, tab))
    if routing is None:
        idx, w, _ = router_b(x, gate[0], gate[1], k, renormalize, tab, win, gate[2] if len(gate) > 2 else None)
    else:
        idx, w = routing[0].to(torch.int64), routing[1].to(BF)
    y = _moe_layer_mx(x, idx, w, expert_tables_mx(experts), _act_code(act))
    return y, idx, w


# ============================================================================ block-scaled activations (MX2)
def blockquant(x: torch.Tensor):
    """x [T, K] -> (q int8 [T, K], ka int32 [T, K/32]): per 32-wide block, ka = the least k with
    127 * 2^k >= max |x| (clamped to [-126, 127], -126 for a zero block), q = rint(x / 2^ka)."""
    return ops.blockquant(x)


def int_mm_mx2(q: torch.Tensor, ka: torch.Tensor, m2: torch.Tensor, kexp: torch.Tensor) -> torch.Tensor:
    """q int8 [T, K], ka int32 [T, nb]; m2 int8 [N, K], kexp uint8 [N, nb] -> binary32 [T, N]: per
    block s (exact), acc = fl32(acc + fl32(s * fl32(2^(ka + kexp - 128)))) in ascending order."""
    return ops.gemm_mx2(q, ka, m2, kexp, 0)


def expert_block_mx2(x_rows, w13, w2, act, b13=None, b2=None):
    """blockquant -> int_mm_mx2 -> bfr (+ b13) -> act -> blockquant(bf16 h) -> int_mm_mx2 -> bfr (+ b2)."""
    q, ka = blockquant(x_rows)
    y = ops.gemm_mx2(q, ka, w13[0], w13[1], 0, bias=b13, epilogue=1)
    I = y.shape[-1] // 2
    h = act(y[:, :I], y[:, I:])
    q2, ka2 = blockquant(h.to(BF))
    return ops.gemm_mx2(q2, ka2, w2[0], w2[1], 0, bias=b2, epilogue=1)


def moe_forward_mx2(x, gate, experts, k, renormalize, tab, win, act, routing=None, logits=None):
    """As moe_forward_mx with block-scaled activations (no per-row scale; epilogues bfr(acc) + b).
    experts[e] = ((m2_13, kexp_13), (m2_2, kexp_2), b13 | None, b2 | None) or an ExpertTablesMX.
    logits: as moe_forward's."""
    if logits is not None:
        return _moe_layer_mx(x, None, None, expert_tables_mx(experts), _act_code(act), wfmt=2,
                             route=(logits, k, renormalize, tab))
    if routing is None:
        idx, w, _ = router_b(x, gate[0], gate[1], k, renormalize, tab, win, gate[2] if len(gate) > 2 else None)
    else:
        idx, w = routing[0].to(torch.int64), routing[1].to(BF)
    y = _moe_layer_mx(x, idx, w, expert_tables_mx(experts), _act_code(act), wfmt=2)
    return y, idx, w
