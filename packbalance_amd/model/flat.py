"""Flat parameter storage for the training harness: one fp32 buffer for the
master weights, one for their gradients, and one compute-dtype copy (bf16
under autocast) of the weights for the matmuls.

Every ``nn.Parameter`` of the model becomes a view into the master buffer
(``p.data``) and its ``.grad`` a view into the gradient buffer, so

* the step's optimizer and gradient clipping run over ONE tensor (a single
  ``nn.Parameter`` over the whole master buffer, ``FlatParams.param``);
* parameters listed as a group (q/k/v, gate/up) are adjacent, so their
  weights, bf16 copies and gradients are also one ``[sum rows, cols]`` matrix
  each -- one fused GEMM instead of three or two;
* matmul backward passes accumulate weight gradients in fp32 straight into
  the gradient buffer (no bf16 dW, no cast, no separate add per micro-batch).

Micro-batches run concurrently (one stream each) must not add into one
gradient buffer at once, so the store can hold several gradient SLOTS: rows
of one ``[slots, n]`` buffer, slot 0 being ``grad`` (what every ``p.grad``
views).  Inside ``accumulate_into(i)`` the weight-gradient targets handed out
by ``grad_of`` are slot ``i``'s; the fused optimizer step sums the slots into
slot 0 before clipping.

The compute-dtype copy is what torch's autocast computes on the fly (each
fp32 weight rounded to bf16 once per autocast region); here it is one cast
kernel over the whole buffer, run by ``refresh`` -- by the model on every
forward, or once per step inside ``hold()`` unless the optimizer already
wrote it with the update (``mark_fresh``).
"""

from __future__ import annotations

import contextlib

import torch
from torch import nn

from packbalance_amd import _native as N

_ALIGN = 64  # elements: every non-grouped parameter and group starts 256-byte aligned


def _align(n: int) -> int:
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


class FlatParams:
    def __init__(self, model: nn.Module, groups: list[list[nn.Parameter]] = (),
                 grad_slots: int = 1) -> None:
        if grad_slots < 1:
            raise ValueError(f"grad_slots must be >= 1, got {grad_slots}")
        named = list(model.named_parameters())
        if not named:
            raise ValueError("model has no parameters")
        dev = named[0][1].device
        follows = {}  # id(param) -> previous member of its group
        for g in groups:
            shapes = {tuple(p.shape[1:]) for p in g}
            if len(shapes) != 1:
                raise ValueError("grouped parameters must share their trailing shape")
            for prev, p in zip(g, g[1:]):
                follows[id(p)] = id(prev)
        off = 0
        self._off: dict[int, tuple[int, torch.Size]] = {}
        last_id = None
        for _, p in named:
            if id(p) in follows:
                if follows[id(p)] != last_id:
                    raise ValueError("grouped parameters must be registered consecutively")
            else:
                off = _align(off)
            self._off[id(p)] = (off, p.shape)
            off += p.numel()
            last_id = id(p)
        total = _align(off)
        self.device = dev
        self.master = torch.zeros(total, dtype=torch.float32, device=dev)
        self._grads = torch.zeros((grad_slots, total), dtype=torch.float32, device=dev)
        self.grad = self._grads[0]
        self._slot = 0
        self._params = [p for _, p in named]
        with torch.no_grad():
            for p in self._params:
                v = self._view(self.master, p)
                v.copy_(p.detach().float())
                gv = self._view(self.grad, p)
                if p.grad is not None:
                    gv.copy_(p.grad)
                p.data = v
                p.grad = gv
        self._gviews = [p.grad for p in self._params]
        self.param = nn.Parameter(self.master)
        self.param.grad = self.grad
        self._shadow: dict[torch.dtype, torch.Tensor] = {}
        self._cache: dict[tuple, torch.Tensor] = {}
        self._tcache: dict[tuple, tuple[int, torch.Tensor]] = {}
        self._held = False
        self._fresh: set[torch.dtype] = set()  # copies known to equal the master weights
        self.refreshes = 0  # number of compute-copy rewrites (host-side counter)

    # ------------------------------------------------------------ views
    def _view(self, buf: torch.Tensor, p: nn.Parameter) -> torch.Tensor:
        o, shape = self._off[id(p)]
        return buf[o:o + p.numel()].view(shape)

    def owns(self, model: nn.Module) -> bool:
        """True while every parameter still lives in this store (no .to(), no re-assign)."""
        ps = [p for p in model.parameters()]
        if len(ps) != len(self._params):
            return False
        for p in (ps[0], ps[-1]):
            if id(p) not in self._off or p.data_ptr() != self._view(self.master, p).data_ptr():
                return False
        return True

    def _group(self, buf: torch.Tensor, params, key) -> torch.Tensor:
        ck = (key, tuple(id(p) for p in params))
        hit = self._cache.get(ck)
        if hit is not None:
            return hit
        first, last = params[0], params[-1]
        o0, shape = self._off[id(first)]
        o1 = self._off[id(last)][0] + last.numel()
        rows = sum(p.shape[0] for p in params)
        v = buf[o0:o1].view((rows,) + tuple(shape[1:]))
        self._cache[ck] = v
        return v

    def weight(self, params, dtype: torch.dtype) -> torch.Tensor:
        """The compute-dtype weights of ``params`` (adjacent), as one matrix."""
        if dtype == torch.float32:
            return self._group(self.master, params, "master")
        return self._group(self._shadow_buf(dtype), params, dtype)

    def transposed(self, groups, dtype: torch.dtype) -> torch.Tensor:
        """[len(groups), cols, rows]: each group's compute-dtype weight matrix transposed.

        The groups (one per layer, e.g. every layer's stacked q/k/v) must have one
        shape and sit at a constant stride in the store, so one strided copy
        transposes them all.  Rebuilt into the same buffer whenever the compute
        copy was rewritten.  (hipBLASLt runs the input-gradient products
        dx = dy W fastest with W given transposed.)"""
        key = (dtype, tuple(id(g[0]) for g in groups))
        hit = self._tcache.get(key)
        if hit is not None and hit[0] == self.refreshes:
            return hit[1]
        buf = self.master if dtype == torch.float32 else self._shadow_buf(dtype)
        first = [self._off[id(g[0])][0] for g in groups]
        rows = sum(p.shape[0] for p in groups[0])
        cols = int(groups[0][0].shape[1])
        stride = first[1] - first[0] if len(groups) > 1 else rows * cols
        for i, g in enumerate(groups):
            if first[i] != first[0] + i * stride or sum(p.shape[0] for p in g) != rows:
                raise ValueError("transposed(): groups must share a shape and a constant stride")
        dst = hit[1] if hit is not None else torch.empty((len(groups), cols, rows), dtype=buf.dtype,
                                                          device=buf.device)
        N.require_device(buf, op="FlatParams.transposed")
        N.call("pb_transpose_batched", buf.data_ptr() + first[0] * buf.element_size(), stride, cols,
               dst.data_ptr(), len(groups), rows, cols, buf.element_size(), N.stream_ptr(buf))
        self._tcache[key] = (self.refreshes, dst)
        return dst

    def grad_of(self, params) -> torch.Tensor:
        """The fp32 gradient of ``params`` (adjacent), as one matrix, in the active slot."""
        return self._group(self._grads[self._slot], params, ("grad", self._slot))

    @property
    def grad_slots(self) -> int:
        return self._grads.shape[0]

    @property
    def grad_slot_stride(self) -> int:
        """Elements from one gradient slot to the next."""
        return self._grads.stride(0)

    @contextlib.contextmanager
    def accumulate_into(self, slot: int):
        """Weight gradients of the forwards run inside the block go to ``slot``
        (their backward passes keep that target whenever they run)."""
        if not 0 <= slot < self.grad_slots:
            raise ValueError(f"gradient slot {slot} out of range [0, {self.grad_slots})")
        prev, self._slot = self._slot, slot
        try:
            yield
        finally:
            self._slot = prev

    # ------------------------------------------------------------ compute copy
    def _shadow_buf(self, dtype: torch.dtype) -> torch.Tensor:
        buf = self._shadow.get(dtype)
        if buf is None:
            buf = torch.empty(self.master.numel(), dtype=dtype, device=self.device)
            self._shadow[dtype] = buf
            self._held = False
        return buf

    def refresh(self, dtype: torch.dtype) -> bool:
        """Round the master weights to ``dtype`` (no-op for fp32 or inside ``hold``).

        Returns True when the copy was rewritten."""
        if dtype == torch.float32:
            if not self._held:
                self.refreshes += 1  # fp32 "copies" are the masters: derived views go stale
            return False
        if self._held:
            return False
        with torch.no_grad():
            self._shadow_buf(dtype).copy_(self.master)
        self.mark_fresh(dtype)
        return True

    def mark_fresh(self, dtype: torch.dtype) -> None:
        """The ``dtype`` copy was just rewritten from the master weights (by ``refresh``
        or by an optimizer step that writes it)."""
        self._fresh = {dtype}
        self.refreshes += 1

    def invalidate(self) -> None:
        """The master weights were changed outside the optimizer: the next ``hold``
        refreshes the copy."""
        self._fresh = set()

    @contextlib.contextmanager
    def hold(self, dtype: torch.dtype):
        """Refresh the copy unless it is known fresh, then keep it for every forward
        inside the block (the master weights must not change inside it)."""
        if dtype not in self._fresh:
            self.refresh(dtype)
        self._held = dtype != torch.float32
        try:
            yield
        finally:
            self._held = False

    # ------------------------------------------------------------ gradients
    def attach_grads(self) -> None:
        """Point every ``p.grad`` back at its view (after ``zero_grad(set_to_none=True)``
        or a user assignment), keeping any gradient it held."""
        with torch.no_grad():
            for p, v in zip(self._params, self._gviews):
                g = p.grad
                if g is None:
                    v.zero_()
                elif g.data_ptr() != v.data_ptr():
                    v.copy_(g)
                else:
                    continue
                p.grad = v
            if self.param.grad is None or self.param.grad.data_ptr() != self.grad.data_ptr():
                self.param.grad = self.grad

    def zero_grad(self) -> None:
        """Zero every gradient slot (one fill)."""
        self._grads.zero_()
