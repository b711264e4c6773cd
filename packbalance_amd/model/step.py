"""The packed training step of the benchmark harness, eager or as one HIP graph.

Semantics of the reference's ``profiling/bench_train.py:101-118``: for each
pack of the step (one micro-batch each) build the document block mask, run
the forward and ``(loss / step_tokens).backward()`` under bf16 autocast; then
``clip_grad_norm_(1.0)`` and a fused AdamW step.

The step's gradient is the sum of the packs' gradients, however the packs are
grouped into micro-batches, so ``packs_per_micro_batch`` > 1 runs several
packs as one [k, S] batch (one forward and one backward over k*S tokens:
GEMMs k times taller, a k-times larger attention grid, k times fewer
launches) -- the same gradient up to the order of fp32 additions.  The
document mask of a micro-batch is built as the attention kernels' tile plans
(``DocPlans``); the FlexAttention tables the reference builds for its
attention have no reader here.

The parameters live in the model's flat store (``FlatParams``): the step
zeroes the one gradient buffer, runs every micro-batch on one bf16 copy of
the weights (``hold``), and clips and updates the flat buffer with the fused
``FlatAdamW`` -- the same arithmetic as ``clip_grad_norm_`` plus fused AdamW
over the per-tensor list (uniform hyper-parameters, element-wise update) --
whose update also writes the next step's bf16 copy.

With a ``DeviceTokenStore`` the step's packs are built on the device
(``PackBuilder``: input ids, labels, positions and document ids from the
store in HBM and a small per-step segment table) as the first work of the
step -- the part of the reference's timed step that loads and copies the
micro-batches (``bench_train.py:103-111``) -- and the step's token count
comes from the same table, so a replay needs only the table's copy.

With ``streams > 1`` the micro-batches run concurrently, micro-batch i on
stream i % streams: at 2048 tokens a micro-batch's kernels fill only part of
the GPU, so the chains overlap.  Each stream adds its weight gradients into
its own gradient slot of the flat store (no two streams write one buffer),
the shared weight copies are built on the step's stream before the fork, and
the optimizer's norm pass sums the slots -- the same gradient as the
sequential step up to the order of fp32 additions.  Every gradient write
happens in a backward pass, so the slots are zeroed on a side stream
while the forwards run, and each backward first waits for that fill (also
when the micro-batches run one after another on the step's stream).

``keep_logits_bytes`` (default 1 GiB) lets each micro-batch's LM-head forward
keep its bf16 logits for the backward when they fit in that many bytes
(``fused_ce.logits_budget``; 262 MB per [2, 2048] micro-batch at cfg2): the
same numerics without the backward's logits GEMM, the LM-head forward and
backward being adjacent in the pass.  0 recomputes the logits in the
backward, as the reference's chunked CE does.  cfg2, alternating runs on one
box (40 timed steps each): 706.8k against 691.5k tok/s.

``capture`` records that whole sequence once into a HIP graph on static
device buffers (every hot-path op is capture-safe: no host synchronisation,
device-resident grad scale, all workspaces from the caching allocator);
``replay`` copies the next step's packs -- already resident in HBM -- into
those buffers and replays it, so the ~5k kernel launches of a step cost one
graph launch.  ``loss_sum`` and ``grad_norm`` hold the last step's summed
loss and pre-clip gradient norm for checking replays against eager steps.
"""

from __future__ import annotations

import torch

from packbalance_amd.data.device_packs import DeviceTokenStore, PackBuilder
from packbalance_amd.kernels.fused_ce import logits_budget
from packbalance_amd.model import layers as L
from packbalance_amd.model.attention import DocPlans
from packbalance_amd.model.llama import LlamaForCausalLM
from packbalance_amd.model.optim import FlatAdamW


class TrainStep:
    def __init__(self, cfg, dev, packs_per_step: int = 4, seq_len: int | None = None,
                 seed: int = 0, lr: float = 3e-4, store: DeviceTokenStore | None = None,
                 streams: int = 1, packs_per_micro_batch: int = 1,
                 keep_logits_bytes: int = 1 << 30):
        self.cfg, self.dev = cfg, dev
        self.keep_logits_bytes = int(keep_logits_bytes)
        seq_len = seq_len or cfg.max_seq_len
        if seq_len > cfg.max_seq_len:
            # positions restart per document, so they stay below seq_len: within
            # the RoPE cache, which a captured step cannot check on the host
            raise ValueError(f"seq_len {seq_len} exceeds the model's max_seq_len {cfg.max_seq_len}")
        k = int(packs_per_micro_batch)
        if k < 1 or packs_per_step % k:
            raise ValueError(f"packs_per_micro_batch {k} does not divide packs_per_step "
                             f"{packs_per_step}")
        self.k = k
        n_micro = packs_per_step // k
        streams = max(1, min(int(streams), n_micro))
        torch.manual_seed(seed)
        self.model = LlamaForCausalLM(cfg).to(dev)
        self.model.train()
        self.flat = self.model.flat_parameters(grad_slots=streams)
        self.streams = [torch.cuda.Stream(dev) for _ in range(streams)] if streams > 1 else []
        # The gradient slots are zeroed on a side stream while the (first) forwards
        # run: every gradient write happens in a backward.
        self.zero_stream = torch.cuda.Stream(dev)
        self.stream_loss = torch.zeros(streams, dtype=torch.float32, device=dev)
        self.opt = FlatAdamW(self.flat, lr=lr, betas=(0.9, 0.95), weight_decay=0.1,
                             max_grad_norm=1.0, copy_dtype=torch.bfloat16)

        def z():
            return torch.zeros((k, seq_len), dtype=torch.int64, device=dev)

        self.builder = None
        if store is not None:
            self.builder = PackBuilder(store, packs_per_step, seq_len)
            out = self.builder.outputs
            self.static = [{key: t[j * k:(j + 1) * k] for key, t in out.items()}
                           for j in range(n_micro)]
        else:
            self.static = [dict(input_ids=z(), labels=z(), position_ids=z(), doc_ids=z())
                           for _ in range(n_micro)]
        self.step_tokens = torch.ones((), dtype=torch.float32, device=dev)
        self.loss_sum = torch.zeros((), dtype=torch.float32, device=dev)
        self.grad_norm = torch.zeros((), dtype=torch.float32, device=dev)
        self.graph = None

    def _body(self, batches, step_tokens, build: bool = False) -> None:
        if build:  # the step's packs from the device token store
            self.builder.launch()
            self.step_tokens.copy_(self.builder.useful_count)
        self.loss_sum.zero_()
        self.flat.attach_grads()
        with torch.autocast("cuda", dtype=torch.bfloat16), self.flat.hold(torch.bfloat16):
            if self.streams:
                self._concurrent(batches, step_tokens)
            else:
                main = torch.cuda.current_stream(self.dev)
                zs = self.zero_stream
                zs.wait_stream(main)
                with torch.cuda.stream(zs):
                    self.flat.zero_grad()
                for i, b in enumerate(batches):
                    self._micro_batch(b, step_tokens, self.loss_sum,
                                      grads_ready=zs if i == 0 else None)
                main.wait_stream(zs)
        self.grad_norm.copy_(self.opt.step())

    def _micro_batch(self, b, step_tokens, loss_acc, grads_ready=None) -> None:
        bm = DocPlans(b["doc_ids"])
        with logits_budget(self.keep_logits_bytes):
            loss = self.model(b["input_ids"], b["labels"], b["position_ids"], b["doc_ids"],
                              block_mask=bm)
        if grads_ready is not None:
            torch.cuda.current_stream(self.dev).wait_stream(grads_ready)
        (loss / step_tokens).backward()
        loss_acc += loss.detach()

    def _concurrent(self, batches, step_tokens) -> None:
        """Micro-batch i on stream i % k, weight gradients into slot i % k; the
        slots are zeroed on a side stream that every backward waits for."""
        main = torch.cuda.current_stream(self.dev)
        self.model.prepare(torch.bfloat16)
        self.stream_loss.zero_()
        zs = self.zero_stream
        zs.wait_stream(main)
        with torch.cuda.stream(zs):
            self.flat.zero_grad()
        for s in self.streams:
            s.wait_stream(main)
        with L.wgrad_on_caller_stream():
            for i, b in enumerate(batches):
                j = i % len(self.streams)
                with torch.cuda.stream(self.streams[j]), self.flat.accumulate_into(j):
                    self._micro_batch(b, step_tokens, self.stream_loss[j], grads_ready=zs)
        for s in self.streams:
            main.wait_stream(s)
        main.wait_stream(zs)
        self.loss_sum.copy_(self.stream_loss.sum())

    _KEYS = ("input_ids", "labels", "position_ids", "doc_ids")

    def _as_dicts(self, batch_list):
        """Packs ([1, S] each) grouped into micro-batches of ``k`` ([k, S])."""
        k = self.k
        return [{key: torch.cat([getattr(b, key) for b in batch_list[j:j + k]])
                 for key in self._KEYS} for j in range(0, len(batch_list), k)]

    def eager(self, batch_list) -> None:
        tokens = float(sum(b.useful_tokens for b in batch_list))
        self._body(self._as_dicts(batch_list), tokens)

    def _load(self, batch_list, tokens_dev) -> None:
        for dst, src in zip(self.static, self._as_dicts(batch_list)):
            for key in self._KEYS:
                dst[key].copy_(src[key])
        self.step_tokens.copy_(tokens_dev)

    def capture(self, batch_list, tokens_dev, warmup_steps: int = 2) -> None:
        """Warm up on a side stream (optimizer state, caches), then capture one step."""
        self._load(batch_list, tokens_dev)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup_steps):
                self._body(self.static, self.step_tokens)
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._body(self.static, self.step_tokens)

    def replay(self, batch_list, tokens_dev) -> None:
        self._load(batch_list, tokens_dev)
        self.graph.replay()

    # ---- packs built on the device (needs ``store``): packs are lists of
    # (start, length) segments of the token store, one list per micro-batch.
    def eager_packs(self, packs) -> None:
        self.builder.load(packs)
        self._body(self.static, self.step_tokens, build=True)

    def capture_packs(self, packs, warmup_steps: int = 2) -> None:
        self.builder.load(packs)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup_steps):
                self._body(self.static, self.step_tokens, build=True)
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._body(self.static, self.step_tokens, build=True)

    def replay_packs(self, packs) -> None:
        self.builder.load(packs)
        self.graph.replay()
