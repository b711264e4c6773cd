"""Projection blocks of the decoder with fused weights and fp32 weight-gradient
accumulation (training harness; the hot-path kernels they call keep the
reference API elsewhere).

Each block takes its activations already in the compute dtype (the fused
norms write bf16 directly), multiplies by a compute-dtype weight matrix from
``FlatParams`` and, in backward, ADDS ``dy^T x`` in fp32 into the weight's
slice of the flat gradient buffer (hipBLASLt with an fp32 C/D and beta 1)
instead of returning a bf16 dW for autograd to cast and accumulate.  The
reference (``packbalance/model/llama.py:57-103``) computes the same products
through ``nn.Linear`` under autocast; the differences are fewer roundings:
dW is never rounded to bf16, and the input gradient of a fused projection is
one fp32 sum rounded once (to the input's dtype, which autograd requires)
instead of a sum of separately rounded products.

* ``qkv_rope``: q, k, v from ONE GEMM against the stacked [q; k; v] weight,
  then RoPE on q and k (the gfx950 kernel) -- ``llama.py:89-92``.
* ``gate_up_swiglu``: gate and up from ONE GEMM against the stacked
  [gate; up] weight, SwiGLU (gfx950 kernel, row-strided halves) --
  ``llama.py:57-61`` minus the down projection.
* ``linear``: o_proj and down_proj.
* ``embed``: the token embedding; its backward adds the gradient rows into
  the fp32 table gradient (index_add) instead of building a dense [V, d]
  gradient per micro-batch.

The weight-gradient GEMMs are off the backward's critical path (nothing in
the pass reads them), and at 2048 tokens per micro-batch each GEMM fills only
part of the GPU, so inside a captured HIP graph they run on a side stream
(``WGRAD_SIDE_STREAM``) and overlap the input-gradient chain.  Eagerly they
stay on the caller's stream: there the step is bound by launch overhead and
the cross-stream waits cost more than the overlap returns.  Each one keeps its operands alive until a
join that an autograd final callback queues at the end of the backward pass;
the callback runs on the stream that called ``backward()``, which then waits
for the side stream -- so gradients are complete when ``backward()`` returns,
eagerly or inside a captured HIP graph (where the wait becomes a graph edge).
A caller that already runs micro-batches concurrently on several streams has
the overlap without it and turns it off (``wgrad_on_caller_stream``).

With a ``WgradPlan`` (the model's training forward passes one) the layers
instead leave x and dy in the plan's per-kind stacked buffers, and the plan
adds every layer's dW of a kind in one batched GEMM when the backward ends.
"""

from __future__ import annotations

import contextlib

import torch
import torch.nn.functional as F

from packbalance_amd import _native as N
from packbalance_amd.model.rope import _rope


WGRAD_SIDE_STREAM = True
# The model's training forward hands its layers a WgradPlan (batched dW GEMMs).
def _wgrad_hooks_available() -> bool:
    """The batched weight-gradient plan ends each backward pass with an autograd
    final callback, through two private PyTorch entry points (present in the
    torch 2.10 this build is tested with): the current graph task id and the
    execution engine's ``queue_callback``.  Without them the layers add their
    weight gradients one GEMM at a time."""
    engine = getattr(torch.autograd.Variable, "_execution_engine", None)
    return (callable(getattr(torch._C, "_current_graph_task_id", None))
            and callable(getattr(engine, "queue_callback", None)))


WGRAD_BATCHED = _wgrad_hooks_available()


@contextlib.contextmanager
def wgrad_per_layer():
    """Weight gradients of the forwards run inside the block are added layer by
    layer (one GEMM each, as the backward reaches them) instead of batched."""
    global WGRAD_BATCHED
    prev, WGRAD_BATCHED = WGRAD_BATCHED, False
    try:
        yield
    finally:
        WGRAD_BATCHED = prev


@contextlib.contextmanager
def wgrad_on_caller_stream():
    """Run weight-gradient GEMMs of the backward passes inside the block on the
    stream that runs the rest of the pass."""
    global WGRAD_SIDE_STREAM
    prev, WGRAD_SIDE_STREAM = WGRAD_SIDE_STREAM, False
    try:
        yield
    finally:
        WGRAD_SIDE_STREAM = prev


class _SideStream:
    """A default-priority side stream per device for weight-gradient GEMMs."""

    _by_device: dict[int, "_SideStream"] = {}

    def __init__(self, dev: torch.device) -> None:
        self.stream = torch.cuda.Stream(dev)
        self.keep: list[torch.Tensor] = []
        self.task = None  # autograd graph task whose end joins this stream

    @classmethod
    def of(cls, dev: torch.device) -> "_SideStream":
        idx = dev.index if dev.index is not None else torch.cuda.current_device()
        s = cls._by_device.get(idx)
        if s is None:
            s = cls._by_device[idx] = cls(torch.device("cuda", idx))
        return s

    def run(self, fn, *keep: torch.Tensor) -> None:
        self.stream.wait_stream(torch.cuda.current_stream(self.stream.device))
        with torch.cuda.stream(self.stream):
            fn()
        self.keep.extend(keep)
        task = torch._C._current_graph_task_id()
        if task != self.task:
            self.task = task
            torch.autograd.Variable._execution_engine.queue_callback(self.join)

    def join(self) -> None:
        torch.cuda.current_stream(self.stream.device).wait_stream(self.stream)
        self.keep.clear()
        self.task = None


def _wgrad(g: torch.Tensor, dy: torch.Tensor, x: torch.Tensor) -> None:
    if dy.dtype == torch.float32:
        g.addmm_(dy.t(), x)
    else:
        torch.addmm(g, dy.t(), x, out_dtype=torch.float32, out=g)


def _accumulate_wgrad(g: torch.Tensor, dy: torch.Tensor, x: torch.Tensor) -> None:
    """g (fp32 [N, K]) += dy^T x, with dy [T, N] and x [T, K] in the compute dtype
    (on the side stream during a backward pass, else inline)."""
    if (WGRAD_SIDE_STREAM and dy.is_cuda and torch._C._current_graph_task_id() >= 0
            and torch.cuda.is_current_stream_capturing()):
        _SideStream.of(dy.device).run(lambda: _wgrad(g, dy, x), dy, x)
    else:
        _wgrad(g, dy, x)


class WgradPlan:
    """The weight-gradient products of one forward/backward pass of the decoder,
    one batched GEMM per weight kind.

    At a micro-batch of a few thousand tokens each layer's dW = dy^T x has a
    small output (768 x 768 .. 4096 x 768 at cfg2) and a long reduction, so
    one GEMM fills only a few hundred tiles; the same product for all L layers
    as one strided-batched GEMM fills the GPU (cfg2: 1.8 -> 0.74 ms per
    micro-batch for the four kinds).  The fused layers therefore write the
    inputs x of their projections (forward) and the gradients dy of their
    outputs (backward) into per-kind stacked buffers ``[L, T, cols]`` (layer l
    at block l; the producing kernels write there directly, else the layer
    copies), and record each layer's fp32 gradient target.  When the backward
    pass ends, every kind whose L targets sit at one constant stride in the
    flat gradient buffer gets ONE ``baddbmm`` (g_l += dy_l^T x_l, fp32 output,
    beta 1); any other set of targets is added layer by layer.
    """

    batched_gemms = 0  # batched GEMMs issued by all plans (a host-side counter)
    norm_reduces = 0  # batched norm dw reductions issued by all plans

    def __init__(self, n_layers: int, tokens: int, dims: dict, dtype: torch.dtype,
                 device: torch.device, norms: int = 0, norm_dim: int = 0) -> None:
        self.L, self.T = n_layers, tokens
        self.dims = dict(dims)
        self.x = {k: torch.empty((n_layers, tokens, c), dtype=dtype, device=device)
                  for k, (_, c) in self.dims.items()}
        self.dy = {k: torch.empty((n_layers, tokens, r), dtype=dtype, device=device)
                   for k, (r, _) in self.dims.items()}
        self.g = {k: [None] * n_layers for k in self.dims}
        # RMSNorm weight gradients (``norms`` norms over [tokens, norm_dim] rows): each
        # norm's backward leaves its per-workgroup dw partials in its row here, and
        # the pass's end adds all of them to their fp32 targets in one launch
        # (at cfg2: 25 small reduction launches per micro-batch -> 1).
        self.norm_dim = norm_dim
        self.norm_parts = None
        if norms:
            from packbalance_amd.kernels.rmsnorm import partial_floats

            self.norm_parts = torch.empty((norms, max(1, partial_floats(tokens, norm_dim))),
                                          dtype=torch.float32, device=device)
        self.norm_g = [None] * norms
        self._task = None

    def x_of(self, kind: str, layer: int) -> torch.Tensor:
        return self.x[kind][layer]

    def dy_of(self, kind: str, layer: int) -> torch.Tensor:
        return self.dy[kind][layer]

    @staticmethod
    def _into(slot: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
        """``slot`` holding ``t``'s values (no copy when t already is the slot).

        The slots of a kind are views of one buffer and share its version
        counter, so the copy goes through ``.data`` (no version bump): a copy
        into one layer's slot must not invalidate the tensors other layers
        saved from theirs.  Every slot is written once per pass, before any
        reader of it runs."""
        if t.data_ptr() != slot.data_ptr() or t.shape != slot.shape or t.stride() != slot.stride():
            slot.data.copy_(t)
        return slot

    def add(self, kind: str, layer: int, g: torch.Tensor) -> None:
        """Called from a layer's backward once ``dy_of(kind, layer)`` holds its dy."""
        self.g[kind][layer] = g
        self._queue_flush()

    def norm_partials(self, slot: int) -> torch.Tensor:
        """Norm ``slot``'s dw partial table (filled by its backward)."""
        return self.norm_parts[slot]

    def add_norm(self, slot: int, g: torch.Tensor) -> None:
        """Called from a norm's backward once ``norm_partials(slot)`` holds its partials;
        ``g`` (fp32 [norm_dim]) receives their sum when the pass ends."""
        self.norm_g[slot] = g
        self._queue_flush()

    def _queue_flush(self) -> None:
        task = torch._C._current_graph_task_id()
        if task != self._task:
            self._task = task
            torch.autograd.Variable._execution_engine.queue_callback(self.flush)

    def _batched_target(self, kind: str):
        gs = self.g[kind]
        if any(g is None for g in gs):
            return None
        r, c = self.dims[kind]
        g0 = gs[0]
        if self.L < 2 or g0.shape != (r, c) or g0.stride() != (c, 1):
            return None
        stride = (gs[1].data_ptr() - g0.data_ptr()) // g0.element_size()
        if stride < r * c:
            return None
        for i, g in enumerate(gs):
            if (g.shape != g0.shape or g.stride() != g0.stride()
                    or g.data_ptr() != g0.data_ptr() + i * stride * g0.element_size()):
                return None
        return g0.as_strided((self.L, r, c), (stride, c, 1))

    def _flush_norms(self) -> None:
        from packbalance_amd.kernels.rmsnorm import dw_reduce_batched

        i, n = 0, len(self.norm_g)
        while i < n:  # runs of consecutive registered slots, one launch each
            if self.norm_g[i] is None:
                i += 1
                continue
            j = i
            while j < n and self.norm_g[j] is not None:
                j += 1
            dw_reduce_batched(self.norm_parts[i:j], self.norm_g[i:j], self.T, self.norm_dim)
            WgradPlan.norm_reduces += 1
            i = j
        self.norm_g = [None] * n

    def flush(self) -> None:
        self._task = None
        self._flush_norms()
        for kind in self.dims:
            if all(g is None for g in self.g[kind]):
                continue
            target = self._batched_target(kind)
            if target is not None:
                torch.baddbmm(target, self.dy[kind].transpose(1, 2), self.x[kind],
                              out_dtype=torch.float32, out=target)
                WgradPlan.batched_gemms += 1
            else:
                for i, g in enumerate(self.g[kind]):
                    if g is not None:
                        _wgrad(g, self.dy[kind][i], self.x[kind][i])
            self.g[kind] = [None] * self.L


def _mm(a: torch.Tensor, b: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    if out_dtype == a.dtype:
        return torch.mm(a, b)
    return torch.mm(a, b, out_dtype=out_dtype)


def _rows(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    t = t.reshape(-1, t.shape[-1])
    if t.dtype != dtype:
        t = t.to(dtype)
    return t if t.stride(-1) == 1 else t.contiguous()


def _dx_weight(w: torch.Tensor, wt: torch.Tensor | None) -> torch.Tensor:
    """W for dx = dy W: the transposed copy viewed back (the layout hipBLASLt runs
    fastest for these shapes) when there is one."""
    return w if wt is None else wt.t()


class _Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, g, wt, plan, kind, layer):
        x2 = _rows(x, w.dtype)
        if plan is not None:
            x2 = plan._into(plan.x_of(kind, layer), x2)
            # x2 is the plan's slot: the plan keeps it, outside saved-tensor version checks
            ctx.save_for_backward(w)
        else:
            ctx.save_for_backward(x2, w)
        y = torch.mm(x2, w.t())
        ctx.g, ctx.wt, ctx.x_dtype, ctx.x_shape = g, wt, x.dtype, x.shape
        ctx.plan, ctx.kind, ctx.layer = plan, kind, layer
        return y.view(*x.shape[:-1], w.shape[0])

    @staticmethod
    def backward(ctx, dy):
        plan = ctx.plan
        if plan is not None:
            (w,) = ctx.saved_tensors
            dy2 = plan._into(plan.dy_of(ctx.kind, ctx.layer), _rows(dy, w.dtype))
        else:
            x2, w = ctx.saved_tensors
            dy2 = _rows(dy, w.dtype)
        dx = _mm(dy2, _dx_weight(w, ctx.wt), ctx.x_dtype)
        if plan is not None:
            plan.add(ctx.kind, ctx.layer, ctx.g)
        else:
            _accumulate_wgrad(ctx.g, dy2, x2)
        return dx.view(ctx.x_shape), None, None, None, None, None, None


def linear(x: torch.Tensor, w: torch.Tensor, g: torch.Tensor,
           wt: torch.Tensor | None = None, plan: WgradPlan | None = None,
           kind: str | None = None, layer: int | None = None) -> torch.Tensor:
    """``x @ w.T``; backward returns dx in x's dtype and adds dW into ``g`` (fp32).
    ``wt`` (optional) is ``w`` transposed and contiguous, used for dx.  With a
    ``plan``, x and dy go to its ``kind`` slots of ``layer`` and dW is added by
    the plan's batched GEMM when the backward pass ends."""
    return _Linear.apply(x, w, g, wt, plan, kind, layer)


class _QKVRope(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, g, cos, sin, hq, hkv, hd, wt, plan, layer):
        b, s, dm = x.shape
        x2 = _rows(x, w.dtype)
        if plan is not None:
            x2 = plan._into(plan.x_of("qkv", layer), x2)
        qkv = torch.mm(x2, w.t())  # [T, (hq + 2 hkv) hd]
        nq, nk = hq * hd, hkv * hd
        q = qkv[:, :nq].view(b, s, hq, hd).transpose(1, 2)
        k = qkv[:, nq:nq + nk].view(b, s, hkv, hd).transpose(1, 2)
        v = qkv[:, nq + nk:].view(b, s, hkv, hd).transpose(1, 2)
        qr = torch.empty((b, s, hq, hd), dtype=qkv.dtype, device=x.device).transpose(1, 2)
        kr = torch.empty((b, s, hkv, hd), dtype=qkv.dtype, device=x.device).transpose(1, 2)
        _rope(q, k, qr, kr, cos, sin, 0)
        if plan is not None:
            # x2 is the plan's slot: the plan keeps it, outside saved-tensor version checks
            ctx.save_for_backward(w, cos, sin)
        else:
            ctx.save_for_backward(x2, w, cos, sin)
        ctx.g, ctx.wt, ctx.dims, ctx.x_dtype = g, wt, (b, s, dm, hq, hkv, hd), x.dtype
        ctx.plan, ctx.layer = plan, layer
        return qr, kr, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        plan = ctx.plan
        if plan is not None:
            w, cos, sin = ctx.saved_tensors
        else:
            x2, w, cos, sin = ctx.saved_tensors
        b, s, dm, hq, hkv, hd = ctx.dims
        nq, nk = hq * hd, hkv * hd
        dt = w.dtype
        if plan is not None:
            dqkv = plan.dy_of("qkv", ctx.layer)
        else:
            dqkv = torch.empty((b * s, nq + 2 * nk), dtype=dt, device=w.device)
        oq = dqkv[:, :nq].view(b, s, hq, hd).transpose(1, 2)
        ok = dqkv[:, nq:nq + nk].view(b, s, hkv, hd).transpose(1, 2)
        ov = dqkv[:, nq + nk:].view(b, s, hkv, hd).transpose(1, 2)
        dq = torch.zeros_like(oq) if dq is None else dq.to(dt)
        dk = torch.zeros_like(ok) if dk is None else dk.to(dt)
        if dq.stride(-1) != 1:
            dq = dq.contiguous()
        if dk.stride(-1) != 1:
            dk = dk.contiguous()
        _rope(dq, dk, oq, ok, cos, sin, 1)
        if dv is None:
            ov.zero_()
        elif dv.data_ptr() != ov.data_ptr() or dv.stride() != ov.stride():
            ov.copy_(dv)  # (the attention backward may have written dV here already)
        dx = _mm(dqkv, _dx_weight(w, ctx.wt), ctx.x_dtype)
        if plan is not None:
            plan.add("qkv", ctx.layer, ctx.g)
        else:
            _accumulate_wgrad(ctx.g, dqkv, x2)
        return dx.view(b, s, dm), None, None, None, None, None, None, None, None, None, None


def qkv_rope(x, w, g, cos, sin, hq: int, hkv: int, hd: int, wt: torch.Tensor | None = None,
             plan: WgradPlan | None = None, layer: int | None = None):
    """q [B, hq, S, hd] and k [B, hkv, S, hd] (RoPE applied) and v, from one GEMM
    against the stacked [q; k; v] weight ``w``; backward adds dW into ``g`` (through
    ``plan``'s "qkv" slots of ``layer`` when given)."""
    N.require_device(x, w, op="qkv_rope")
    if x.dim() != 3 or w.shape != ((hq + 2 * hkv) * hd, x.shape[-1]):
        raise ValueError(f"qkv_rope: x {tuple(x.shape)} / w {tuple(w.shape)} do not match "
                         f"hq={hq} hkv={hkv} hd={hd}")
    return _QKVRope.apply(x, w, g, cos, sin, hq, hkv, hd, wt, plan, layer)


class _GateUpSwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, g, wt, plan, layer):
        x2 = _rows(x, w.dtype)
        if plan is not None:
            x2 = plan._into(plan.x_of("gate_up", layer), x2)
        gu = torch.mm(x2, w.t())  # [T, 2F]: gate | up
        t, f2 = gu.shape
        f = f2 // 2
        if plan is not None:  # the down projection's input slot
            a = plan.x_of("down", layer)
        else:
            a = torch.empty((t, f), dtype=gu.dtype, device=gu.device)
        N.call("pb_swiglu_fwd_rows", gu.data_ptr(), f2, gu[:, f:].data_ptr(), f2, a.data_ptr(), f,
               t, f, N.dtype_code(gu), N.stream_ptr(gu))
        if plan is not None:
            # x2 is the plan's slot: the plan keeps it, outside saved-tensor version checks
            ctx.save_for_backward(w, gu)
        else:
            ctx.save_for_backward(x2, w, gu)
        ctx.g, ctx.wt, ctx.x_dtype, ctx.x_shape = g, wt, x.dtype, x.shape
        ctx.plan, ctx.layer = plan, layer
        return a.view(*x.shape[:-1], f)

    @staticmethod
    def backward(ctx, da):
        plan = ctx.plan
        if plan is not None:
            w, gu = ctx.saved_tensors
        else:
            x2, w, gu = ctx.saved_tensors
        t, f2 = gu.shape
        f = f2 // 2
        da2 = _rows(da, gu.dtype)
        dgu = plan.dy_of("gate_up", ctx.layer) if plan is not None else torch.empty_like(gu)
        N.call("pb_swiglu_bwd_rows", gu.data_ptr(), f2, gu[:, f:].data_ptr(), f2, da2.data_ptr(),
               da2.stride(0), dgu.data_ptr(), f2, dgu[:, f:].data_ptr(), f2, t, f,
               N.dtype_code(gu), N.stream_ptr(gu))
        dx = _mm(dgu, _dx_weight(w, ctx.wt), ctx.x_dtype)
        if plan is not None:
            plan.add("gate_up", ctx.layer, ctx.g)
        else:
            _accumulate_wgrad(ctx.g, dgu, x2)
        return dx.view(ctx.x_shape), None, None, None, None, None


def gate_up_swiglu(x: torch.Tensor, w: torch.Tensor, g: torch.Tensor,
                   wt: torch.Tensor | None = None, plan: WgradPlan | None = None,
                   layer: int | None = None) -> torch.Tensor:
    """``silu(x @ Wg.T) * (x @ Wu.T)`` from one GEMM against ``w`` = [Wg; Wu].  With a
    ``plan`` the output is written into its "down" input slot of ``layer`` and dW
    goes through its "gate_up" slots."""
    N.require_device(x, w, op="gate_up_swiglu")
    if w.shape[0] % 2 or w.shape[1] != x.shape[-1]:
        raise ValueError(f"gate_up_swiglu: w {tuple(w.shape)} does not match x {tuple(x.shape)}")
    return _GateUpSwiGLU.apply(x, w, g, wt, plan, layer)


class _Embed(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ids, weight, g):
        ctx.save_for_backward(ids)
        ctx.g = g
        return F.embedding(ids, weight.detach())

    @staticmethod
    def backward(ctx, dout):
        (ids,) = ctx.saved_tensors
        g = ctx.g
        g.index_add_(0, ids.reshape(-1), dout.reshape(-1, g.shape[1]).to(g.dtype))
        return None, None, None


def embed(ids: torch.Tensor, weight: torch.nn.Parameter, g: torch.Tensor) -> torch.Tensor:
    """``weight[ids]``; backward adds the rows of the incoming gradient into ``g``.

    ``weight`` is passed so the output joins the autograd graph; its gradient is
    delivered through ``g`` (the returned gradient is None)."""
    return _Embed.apply(ids, weight, g)
