"""CPU oracle for PackBalance's training hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithms that the gfx950
kernels in ``packbalance_amd`` replace.  It is imported only by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``, and
only as the checker or the timed CPU baseline -- never as a code path of the
product.  Nothing in ``packbalance_amd`` imports it.

Modules (each function cites the reference file:line it follows):
  kernels     RMSNorm, SwiGLU, row CE, linear CE  (packbalance/kernels/*.py)
  attention   document-masked GQA attention, dense-mask and per-document forms
              (packbalance/model/attention.py)
  block_mask  FlexAttention BlockMask tables from doc_ids
              (torch.nn.attention.flex_attention.create_block_mask semantics)
  optim       gradient clipping + AdamW step (torch.nn.utils.clip_grad_norm_ +
              torch.optim.AdamW, as the reference's train loop calls them)
  data        model inputs of packs from a token array (packbalance/data/dataset.py)

How each function is pinned (beyond restating its formula) is listed in
``tests/test_oracle.py``; every oracle function has at least one check there
against a library routine, a golden fixture, a closed form or autograd.
"""
