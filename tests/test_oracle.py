"""Pins for the CPU oracle (runs without a GPU).

Each oracle function is checked against something other than its own
formula: a PyTorch library routine, autograd, a golden fixture produced by
torch's create_block_mask, an independent restatement, or a closed form.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as OA
from oracle import block_mask as OB
from oracle import data as OD
from oracle import kernels as OK
from oracle import optim as OO

GOLDEN = Path(__file__).resolve().parent / "golden" / "block_masks.npz"


# ---------------------------------------------------------------- RMSNorm
def test_rmsnorm_oracle_matches_autograd_and_closed_form() -> None:
    torch.manual_seed(0)
    x = torch.randn(8, 32, dtype=torch.float64)
    w = torch.randn(32, dtype=torch.float64)
    dy = torch.randn(8, 32, dtype=torch.float64)
    eps = 1e-5
    xa = x.clone().requires_grad_(True)
    wa = w.clone().requires_grad_(True)
    ya = xa * torch.rsqrt(xa.pow(2).mean(-1, keepdim=True) + eps) * wa
    ya.backward(dy)
    y, rstd = OK.rmsnorm_fwd(x, w, eps)
    dx, dw = OK.rmsnorm_bwd(dy, x, w, eps)
    torch.testing.assert_close(y, ya.detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dx, xa.grad, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(dw, wa.grad, rtol=1e-10, atol=1e-10)
    # Closed form: a constant row c gives rstd = 1/sqrt(c^2 + eps).
    c = torch.full((1, 16), 3.0, dtype=torch.float64)
    _, r = OK.rmsnorm_fwd(c, torch.ones(16, dtype=torch.float64), eps)
    assert abs(float(r[0]) - 1.0 / math.sqrt(9.0 + eps)) < 1e-15


# ---------------------------------------------------------------- SwiGLU
def test_add_rmsnorm_oracle_matches_autograd() -> None:
    """h = x + delta then RMSNorm: both outputs' gradients reach x and delta summed."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(6, 24, generator=g, dtype=torch.float64, requires_grad=True)
    d = torch.randn(6, 24, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(24, generator=g, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(6, 24, generator=g, dtype=torch.float64)
    dres = torch.randn(6, 24, generator=g, dtype=torch.float64)
    h = x + d
    y = h * torch.rsqrt((h * h).mean(-1, keepdim=True) + 1e-5) * w
    torch.autograd.backward((h, y), (dres, dy))
    oh, oy, _ = OK.add_rmsnorm_fwd(x, d, w, 1e-5)
    torch.testing.assert_close(oh, h.detach())
    torch.testing.assert_close(oy, y.detach())
    ddx, ddw = OK.add_rmsnorm_bwd(dy, dres, oh, w, 1e-5)
    torch.testing.assert_close(ddx, x.grad)
    torch.testing.assert_close(ddx, d.grad)
    torch.testing.assert_close(ddw, w.grad)


def test_swiglu_oracle_matches_autograd() -> None:
    torch.manual_seed(0)
    g = torch.randn(8, 16, dtype=torch.float64, requires_grad=True)
    u = torch.randn(8, 16, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(8, 16, dtype=torch.float64)
    ref = F.silu(g) * u
    ref.backward(dy)
    out = OK.swiglu_fwd(g, u)
    dg, du = OK.swiglu_bwd(g, u, dy)
    torch.testing.assert_close(out, ref.detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dg, g.grad, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(du, u.grad, rtol=1e-10, atol=1e-10)


# ---------------------------------------------------------------- CE
@pytest.mark.parametrize("z_loss", [0.0, 0.01])
def test_linear_ce_oracle_matches_full_ce(z_loss: float) -> None:
    # The reference's own CE test pattern (tests/test_kernels.py:64-81).
    torch.manual_seed(0)
    x = torch.randn(37, 32, dtype=torch.float64)
    w = torch.randn(64, 32, dtype=torch.float64)
    t = torch.randint(0, 64, (37,))
    t[::7] = -100
    x1 = x.clone().requires_grad_(True)
    w1 = w.clone().requires_grad_(True)
    loss = OK.full_ce_reference(x1, w1, t, z_loss)
    loss.backward()
    l2, dx, dw = OK.linear_ce(x, w, t, z_loss_coeff=z_loss)
    # The reference formula takes the z-loss lse through .float() (fp32).
    tol = 1e-10 if z_loss == 0 else 1e-6
    torch.testing.assert_close(l2, loss.detach(), rtol=tol, atol=tol)
    torch.testing.assert_close(dx, x1.grad, rtol=tol, atol=tol)
    torch.testing.assert_close(dw, w1.grad, rtol=tol, atol=tol)


def test_linear_ce_oracle_bf16_logits() -> None:
    """logits_dtype=bf16: the CE of the bf16-rounded product, pinned by F.cross_entropy
    and autograd on logits rounded by torch's own cast (the rounding is a constant for
    the gradient), and different from the unrounded CE when logits are large."""
    torch.manual_seed(3)
    x = torch.randn(29, 24, dtype=torch.float64)
    w = torch.randn(80, 24, dtype=torch.float64) * 2.0
    t = torch.randint(0, 80, (29,))
    t[::6] = -100
    lg = (x @ w.t()).to(torch.bfloat16).to(torch.float64).requires_grad_(True)
    want = torch.nn.functional.cross_entropy(lg, t, ignore_index=-100, reduction="sum")
    want.backward()
    loss, dx, dw = OK.linear_ce(x, w, t, logits_dtype=torch.bfloat16)
    torch.testing.assert_close(loss, want.detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dx, lg.grad @ w, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dw, lg.grad.t() @ x, rtol=1e-12, atol=1e-12)
    l_plain, _, _ = OK.linear_ce(x, w, t)
    assert abs(float(l_plain - loss)) > 1e-6  # the rounding is not a no-op here


def test_ce_rows_special_cases() -> None:
    # Uniform logits: loss = ln V; all-ignored rows: 0; V = 1: loss 0.
    V = 1000
    logits = torch.zeros(3, V, dtype=torch.float64)
    loss, lse, dl = OK.ce_rows(logits, torch.tensor([5, -100, 7]))
    assert abs(float(loss[0]) - math.log(V)) < 1e-12
    assert float(loss[1]) == 0.0 and float(dl[1].abs().sum()) == 0.0
    assert abs(float(dl[0].sum())) < 1e-12  # softmax - onehot sums to 0
    l1, _, _ = OK.ce_rows(torch.randn(4, 1, dtype=torch.float64), torch.zeros(4, dtype=torch.int64))
    assert float(l1.abs().max()) < 1e-12


def test_linear_ce_rejects_row_mismatch() -> None:
    with pytest.raises(ValueError):
        OK.linear_ce(torch.randn(4, 8), torch.randn(5, 8), torch.zeros(3, dtype=torch.int64))


# ---------------------------------------------------------------- attention
def _rope_inputs(seed: int = 0, B: int = 2, H: int = 3, S: int = 11, D: int = 16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, H, S, D, generator=g, dtype=torch.float64)
    theta = torch.rand(B, S, D // 2, generator=g, dtype=torch.float64) * 6.0
    return x, theta


def test_rope_oracle_rotation_invariants() -> None:
    """rope.py:34-42 rotates each (d, d + D/2) pair: pinned by what a rotation fixes."""
    x, th = _rope_inputs()
    c, s = th.cos(), th.sin()
    y = OK.rope(x, c, s)
    half = x.shape[-1] // 2
    # each pair keeps its norm
    torch.testing.assert_close(y[..., :half] ** 2 + y[..., half:] ** 2,
                               x[..., :half] ** 2 + x[..., half:] ** 2)
    # angle 0 is the identity; the inverse undoes the forward
    torch.testing.assert_close(OK.rope(x, torch.ones_like(c), torch.zeros_like(s)), x)
    torch.testing.assert_close(OK.rope(y, c, s, inverse=True), x)
    # angles add: rope(a) then rope(b) == rope(a + b)
    th2 = _rope_inputs(seed=1)[1]
    torch.testing.assert_close(OK.rope(y, th2.cos(), th2.sin()), OK.rope(x, (th + th2).cos(), (th + th2).sin()))
    # a quarter turn maps (x1, x2) -> (-x2, x1), the reference's rotate_half
    q = OK.rope(x, torch.zeros_like(c), torch.ones_like(s))
    torch.testing.assert_close(q, torch.cat((-x[..., half:], x[..., :half]), dim=-1))


def test_rope_oracle_backward_is_the_adjoint() -> None:
    """<rope(x), g> == <x, rope_inverse(g)>: the inverse rotation is the exact backward."""
    x, th = _rope_inputs(seed=2)
    g = _rope_inputs(seed=3)[0]
    c, s = th.cos(), th.sin()
    lhs = (OK.rope(x, c, s) * g).sum()
    rhs = (x * OK.rope(g, c, s, inverse=True)).sum()
    assert abs(float(lhs - rhs)) < 1e-10 * float(x.abs().sum() * g.abs().max())
    # and the transpose of the forward's matrix, column by column on one pair
    e = torch.zeros(1, 1, 1, 2, dtype=torch.float64)
    cs, sn = th[:1, :1, :1].cos(), th[:1, :1, :1].sin()
    cols = []
    for i in range(2):
        e.zero_()
        e[..., i] = 1.0
        cols.append(OK.rope(e, cs, sn).flatten())
    m = torch.stack(cols, dim=1)  # forward matrix
    for i in range(2):
        e.zero_()
        e[..., i] = 1.0
        torch.testing.assert_close(OK.rope(e, cs, sn, inverse=True).flatten(), m.T[:, i])


def test_attention_oracle_matches_sdpa_dense_mask() -> None:
    # The reference's eager-attention test pattern (tests/test_attention.py:14-23).
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 2, 8, 4, dtype=torch.float64) for _ in range(3))
    doc = torch.tensor([[0, 0, 0, 1, 1, 2, 2, 2]])
    mask = OA.dense_mask(doc)
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=mask[:, None])
    out = OA.attention(q, k, v, doc)["out"]
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("semantics", ["flex", "eager"])
def test_attention_oracle_grads_match_autograd_gqa(semantics: str) -> None:
    torch.manual_seed(1)
    B, Hq, Hkv, S, D = 2, 4, 2, 40, 8
    q = torch.randn(B, Hq, S, D, dtype=torch.float64, requires_grad=True)
    k = torch.randn(B, Hkv, S, D, dtype=torch.float64, requires_grad=True)
    v = torch.randn(B, Hkv, S, D, dtype=torch.float64, requires_grad=True)
    doc = torch.tensor([[0] * 13 + [1] * 20 + [-1] * 7, [3] * 5 + [4] * 30 + [5] * 5])
    do = torch.randn(B, Hq, S, D, dtype=torch.float64)
    mask = OA.dense_mask(doc)
    if semantics == "eager":
        mask = mask & (doc[:, :, None] >= 0) & (doc[:, None, :] >= 0)
    ke = k.repeat_interleave(Hq // Hkv, dim=1)
    ve = v.repeat_interleave(Hq // Hkv, dim=1)
    s = (q @ ke.transpose(-1, -2)) / math.sqrt(D)
    s = s.masked_fill(~mask[:, None], -math.inf)
    p = torch.softmax(s, dim=-1)
    p = torch.nan_to_num(p, nan=0.0)  # fully-masked eager pad rows
    ref = p @ ve
    ref.backward(do)
    res = OA.attention(q, k, v, doc, do, semantics=semantics)
    torch.testing.assert_close(res["out"], ref.detach(), rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(res["dq"], q.grad, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(res["dk"], k.grad, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(res["dv"], v.grad, rtol=1e-9, atol=1e-9)


def _dense_attention_grads(q, k, v, doc, do):
    """Dense-mask softmax attention with autograd (flex semantics), float64."""
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    G = q.shape[1] // k.shape[1]
    ke, ve = k.repeat_interleave(G, dim=1), v.repeat_interleave(G, dim=1)
    s = (q @ ke.transpose(-1, -2)) / math.sqrt(q.shape[-1])
    p = torch.softmax(s.masked_fill(~OA.dense_mask(doc)[:, None], -math.inf), dim=-1)
    out = p @ ve
    out.backward(do)
    return out.detach(), p.detach(), ke.detach(), q.grad, k.grad, v.grad


def test_attention_rows_oracle_matches_autograd() -> None:
    """attention_rows (row-local out / lse / dQ) against dense autograd at chosen
    rows, including a document's first row, a pad row and the last row."""
    g = torch.Generator().manual_seed(6)
    B, Hq, Hkv, S, D = 2, 4, 2, 40, 8
    q = torch.randn(B, Hq, S, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, Hkv, S, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, Hkv, S, D, generator=g, dtype=torch.float64)
    do = torch.randn(B, Hq, S, D, generator=g, dtype=torch.float64)
    doc = torch.tensor([[0] * 13 + [1] * 20 + [-1] * 7, [3] * 5 + [4] * 30 + [5] * 5])
    out, p, _, dq, _, _ = _dense_attention_grads(q, k, v, doc, do)
    rows = [torch.tensor([0, 12, 13, 20, 35, 39]), torch.tensor([4, 5, 34, 36])]
    res = OA.attention_rows(q, k, v, doc, do, rows)
    lse = OA.attention(q, k, v, doc)["lse"]
    for b in range(B):
        torch.testing.assert_close(res["out"][b], out[b][:, rows[b]], rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(res["dq"][b], dq[b][:, rows[b]], rtol=1e-10, atol=1e-10)
        torch.testing.assert_close(res["lse"][b], lse[b][:, rows[b]], rtol=1e-12, atol=1e-12)


def test_attention_oracle_delta_out_closed_form() -> None:
    """delta_out = O' shifts each row's delta by eps = rowsum(dO * (O' - O)), so
    dS moves by -P eps: dQ by -scale * eps * (P K), dK by -scale * (P * eps)^T Q
    (summed over the GQA group), dV not at all -- checked against dense
    autograd plus that closed form; delta_out = O reproduces the default."""
    g = torch.Generator().manual_seed(8)
    B, Hq, Hkv, S, D = 1, 4, 2, 24, 8
    q = torch.randn(B, Hq, S, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, Hkv, S, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, Hkv, S, D, generator=g, dtype=torch.float64)
    do = torch.randn(B, Hq, S, D, generator=g, dtype=torch.float64)
    doc = torch.tensor([[0] * 10 + [1] * 14])
    out, p, ke, dq, dk, dv = _dense_attention_grads(q, k, v, doc, do)
    o2 = out + 0.05 * torch.randn(out.shape, generator=g, dtype=torch.float64)
    eps = (do * (o2 - out)).sum(-1, keepdim=True)
    sc = 1.0 / math.sqrt(D)
    want_dq = dq - sc * eps * (p @ ke)
    want_dk = dk - sc * ((p * eps).transpose(-1, -2) @ q).reshape(B, Hkv, Hq // Hkv, S, D).sum(2)
    res = OA.attention(q, k, v, doc, do, delta_out=o2)
    torch.testing.assert_close(res["dq"], want_dq, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(res["dk"], want_dk, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(res["dv"], dv, rtol=1e-10, atol=1e-10)
    same = OA.attention(q, k, v, doc, do, delta_out=out)
    torch.testing.assert_close(same["dq"], dq, rtol=1e-10, atol=1e-10)


def test_attention_oracle_special_cases() -> None:
    # Every token its own document: softmax over one key, out == v (GQA-mapped).
    torch.manual_seed(2)
    q = torch.randn(1, 4, 6, 8, dtype=torch.float64)
    k = torch.randn(1, 2, 6, 8, dtype=torch.float64)
    v = torch.randn(1, 2, 6, 8, dtype=torch.float64)
    out = OA.attention(q, k, v, torch.arange(6)[None])["out"]
    torch.testing.assert_close(out, v.repeat_interleave(2, dim=1), rtol=0, atol=1e-15)
    # Identical keys: uniform causal average of the values of the document.
    k1 = torch.zeros(1, 1, 5, 8, dtype=torch.float64)
    v1 = torch.arange(5, dtype=torch.float64)[None, None, :, None].expand(1, 1, 5, 8)
    o1 = OA.attention(torch.randn(1, 1, 5, 8, dtype=torch.float64), k1, v1, torch.zeros(1, 5))["out"]
    want = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0], dtype=torch.float64)
    torch.testing.assert_close(o1[0, 0, :, 0], want, rtol=0, atol=1e-12)


def test_attention_flops_single_doc() -> None:
    f = OA.attention_flops([8192], 128, 32)
    assert f["pairs"] == 33_558_528
    assert abs(f["fwd"] + f["bwd"] - 1.649e12) / 1.649e12 < 1e-3  # one dense 8192-token pack, Hq=32, D=128


# ---------------------------------------------------------------- block tables
def _golden():
    z = np.load(GOLDEN)
    for name in z["layouts"]:
        yield str(name), z


def test_block_mask_oracle_matches_torch_golden() -> None:
    n = 0
    for name, z in _golden():
        doc = z[f"{name}/doc_ids"]
        heads = int(z[f"{name}/heads"])
        tabs, block = OB.build_doc_block_tables(doc, heads)
        assert block == int(z[f"{name}/block"]), name
        for t in OB.TABLE_NAMES:
            np.testing.assert_array_equal(tabs[t], z[f"{name}/{t}"], err_msg=f"{name}:{t}")
        # The closed-form restatement must agree too.
        closed = OB.tables_closed(doc, heads, block)
        for t in OB.TABLE_NAMES:
            np.testing.assert_array_equal(closed[t], z[f"{name}/{t}"], err_msg=f"closed {name}:{t}")
        n += 1
    assert n >= 15


def test_block_mask_known_answer() -> None:
    # One document of 256 tokens (checked against torch when the fixture was made).
    tabs, block = OB.build_doc_block_tables(np.zeros(256, dtype=np.int64), 1)
    assert block == 128
    assert tabs["kv_num_blocks"][0, 0].tolist() == [1, 1]
    assert tabs["kv_indices"][0, 0].tolist() == [[0, 1], [1, 0]]
    assert tabs["full_kv_num_blocks"][0, 0].tolist() == [0, 1]
    assert tabs["full_kv_indices"][0, 0].tolist() == [[0, 1], [0, 1]]
    assert tabs["full_q_num_blocks"][0, 0].tolist() == [1, 0]
    assert tabs["full_q_indices"][0, 0].tolist() == [[1, 0], [0, 1]]


@pytest.mark.parametrize("seed", range(6))
def test_block_mask_dense_and_closed_agree(seed: int) -> None:
    rng = np.random.default_rng(seed)
    s = int(rng.integers(1, 700))
    block = int(rng.choice([32, 64, 128]))
    doc = np.sort(rng.integers(0, max(1, s // 20), s))
    if seed % 2:
        doc = rng.permutation(doc)  # non-contiguous documents
    if seed % 3 == 0 and s > 4:
        doc[-3:] = -1
    np.testing.assert_array_equal(OB.classify_dense(doc, block), OB.classify_closed(doc, block))


def test_block_mask_rejects_batch() -> None:
    with pytest.raises(ValueError):
        OB.build_doc_block_tables(np.zeros((2, 8), dtype=np.int64), 1)


# ---------------------------------------------------------------- clip + AdamW
@pytest.mark.parametrize("max_norm", [1.0, 0.0, 50.0])
def test_clip_adamw_oracle_matches_torch(max_norm) -> None:
    """Five steps against torch's own clip_grad_norm_ + AdamW (float64, single-tensor
    path); grads are scaled so clipping is active on some steps and not on others."""
    rng = np.random.default_rng(0)
    n = 1001
    p0 = rng.standard_normal(n) * 0.02
    tp = torch.nn.Parameter(torch.tensor(p0.copy()))
    opt = torch.optim.AdamW([tp], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                            foreach=False, fused=False)
    p, m, v = p0.copy(), np.zeros(n), np.zeros(n)
    step = 0
    for k in range(5):
        g = rng.standard_normal(n) * (0.01 if k % 2 else 0.2)
        tp.grad = torch.tensor(g.copy())
        tnorm = float(torch.nn.utils.clip_grad_norm_([tp], max_norm)) if max_norm > 0 else \
            float(tp.grad.norm())
        opt.step()
        step, norm = OO.clip_adamw_step(p, g, m, v, step, lr=3e-4, betas=(0.9, 0.95), eps=1e-8,
                                        weight_decay=0.1, max_norm=max_norm)
        assert step == k + 1
        assert abs(norm - tnorm) <= 1e-12 * tnorm
        np.testing.assert_allclose(p, tp.detach().numpy(), rtol=1e-12, atol=1e-15)
        st = opt.state[tp]
        np.testing.assert_allclose(m, st["exp_avg"].numpy(), rtol=1e-12, atol=1e-18)
        np.testing.assert_allclose(v, st["exp_avg_sq"].numpy(), rtol=1e-12, atol=1e-20)


# ---------------------------------------------------------------- pack tensors
def test_pack_tensors_oracle_known_answers() -> None:
    """Worked by hand from dataset.py:33-76: two documents packed into 8 slots, and
    the padded form with one document per 4-token row."""
    tokens = np.array([10, 11, 12, 13, 14, 15, 16], dtype=np.uint32)
    got = OD.pack_tensors(tokens, [[(0, 3), (4, 2)]], 8, pad_token_id=7)
    assert got["input_ids"].tolist() == [[10, 11, 12, 14, 15, 7, 7, 7]]
    assert got["labels"].tolist() == [[11, 12, -100, 15, -100, -100, -100, -100]]
    assert got["position_ids"].tolist() == [[0, 1, 2, 0, 1, 0, 0, 0]]
    assert got["doc_ids"].tolist() == [[0, 0, 0, 1, 1, -1, -1, -1]]
    pad = OD.pack_tensors(tokens, [[(1, 3), (6, 1)]], 4, rows=2, pad_token_id=0)
    assert pad["input_ids"].tolist() == [[11, 12, 13, 0, 16, 0, 0, 0]]
    assert pad["labels"].tolist() == [[12, 13, -100, -100, -100, -100, -100, -100]]
    assert pad["position_ids"].tolist() == [[0, 1, 2, 0, 0, 0, 0, 0]]
    assert pad["doc_ids"].tolist() == [[0, 0, 0, 0, 1, 1, 1, 1]]
    with pytest.raises(ValueError):
        OD.pack_tensors(tokens, [[(0, 5), (0, 4)]], 8)


def test_pack_tensors_oracle_reference_invariants() -> None:
    """The checks of the reference's tests/test_dataset.py:17-42 on random packs."""
    rng = np.random.default_rng(3)
    tokens = rng.integers(0, 50000, size=5000).astype(np.uint32)
    packs = []
    for _ in range(6):
        segs, used = [], 0
        while True:
            n = int(rng.integers(1, 120))
            if used + n > 512:
                break
            segs.append((int(rng.integers(0, 5000 - n)), n))
            used += n
        packs.append(segs)
    got = OD.pack_tensors(tokens, packs, 512)
    for p, segs in enumerate(packs):
        off = 0
        for seg_id, (start, n) in enumerate(segs):
            toks = tokens[start:start + n].astype(np.int64)
            np.testing.assert_array_equal(got["input_ids"][p, off:off + n], toks)
            np.testing.assert_array_equal(got["labels"][p, off:off + n - 1], toks[1:])
            assert got["labels"][p, off + n - 1] == -100
            np.testing.assert_array_equal(got["position_ids"][p, off:off + n], np.arange(n))
            assert (got["doc_ids"][p, off:off + n] == seg_id).all()
            off += n
        assert (got["labels"][p, off:] == -100).all() and (got["doc_ids"][p, off:] == -1).all()


# ---------------------------------------------------------------- model (oracle/model.py)
def _tiny_model(seed: int = 0, vocab: int = 37, z: float = 0.0):
    """A 2-layer GQA model in float64 with the parameter names oracle/model.py reads."""
    from types import SimpleNamespace

    cfg = SimpleNamespace(vocab_size=vocab, d_model=24, n_layers=2, n_heads=4, n_kv_heads=2,
                          d_ff=40, rope_theta=10000.0, norm_eps=1e-5, ce_chunk_size=5,
                          z_loss_coeff=z)
    g = torch.Generator().manual_seed(seed)
    hd = cfg.d_model // cfg.n_heads
    shapes = {"embed_tokens.weight": (vocab, cfg.d_model), "norm.weight": (cfg.d_model,)}
    for i in range(cfg.n_layers):
        p = f"layers.{i}."
        shapes.update({
            p + "input_layernorm.weight": (cfg.d_model,),
            p + "post_attention_layernorm.weight": (cfg.d_model,),
            p + "self_attn.q_proj.weight": (cfg.n_heads * hd, cfg.d_model),
            p + "self_attn.k_proj.weight": (cfg.n_kv_heads * hd, cfg.d_model),
            p + "self_attn.v_proj.weight": (cfg.n_kv_heads * hd, cfg.d_model),
            p + "self_attn.o_proj.weight": (cfg.d_model, cfg.n_heads * hd),
            p + "mlp.gate_proj.weight": (cfg.d_ff, cfg.d_model),
            p + "mlp.up_proj.weight": (cfg.d_ff, cfg.d_model),
            p + "mlp.down_proj.weight": (cfg.d_model, cfg.d_ff),
        })
    params = {}
    for n, shp in shapes.items():
        t = torch.randn(*shp, generator=g, dtype=torch.float64)
        t = 1.0 + 0.1 * t if len(shp) == 1 else 0.3 * t
        params[n] = t.requires_grad_(True)
    return cfg, params


def _pack(docs: list[torch.Tensor], seq_len: int):
    """dataset.py:33-76 conventions for one pack of token documents."""
    ids = torch.zeros(1, seq_len, dtype=torch.int64)
    lab = torch.full((1, seq_len), -100, dtype=torch.int64)
    pos = torch.zeros(1, seq_len, dtype=torch.int64)
    doc = torch.full((1, seq_len), -1, dtype=torch.int64)
    off = 0
    for d, toks in enumerate(docs):
        n = toks.numel()
        ids[0, off:off + n] = toks
        lab[0, off:off + n - 1] = toks[1:]
        pos[0, off:off + n] = torch.arange(n)
        doc[0, off:off + n] = d
        off += n
    return ids, lab, pos, doc


@pytest.mark.parametrize("z", [0.0, 0.01])
def test_model_oracle_packed_equals_isolated_documents(z: float) -> None:
    """The invariant of the reference's tests/test_attention.py:26-55: a pack of
    documents (positions restarting at 0, pad tail) gives every document exactly
    what it gets alone.  Checked per document (labels of the other documents
    ignored), for the loss and for every parameter gradient."""
    from oracle import model as OM

    cfg, params = _tiny_model(z=z)
    g = torch.Generator().manual_seed(7)
    docs = [torch.randint(0, cfg.vocab_size, (n,), generator=g) for n in (6, 11, 1, 4)]
    ids, lab, pos, doc = _pack(docs, 26)
    # The z-loss term takes lse in fp32 (reference.py:45), summed in another order.
    ltol = 1e-7 if z else 1e-12
    off = 0
    for d, toks in enumerate(docs):
        n = toks.numel()
        only = torch.full_like(lab, -100)
        only[0, off:off + n] = lab[0, off:off + n]
        packed = OM.loss(params, cfg, ids, only, pos, doc)
        gp = torch.autograd.grad(packed, list(params.values()))
        i1, l1, p1, d1 = _pack([toks], n)
        alone = OM.loss(params, cfg, i1, l1, p1, d1)
        ga = torch.autograd.grad(alone, list(params.values()))
        torch.testing.assert_close(packed, alone, rtol=ltol, atol=ltol)
        # RMSNorm runs in fp32 (reference.py:10 takes x.float()), so the weight
        # gradients' row sums round at fp32 level in a different order.
        for a, b in zip(gp, ga):
            torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6)
        off += n
    # and the whole pack's loss is the sum over its documents
    total = OM.loss(params, cfg, ids, lab, pos, doc)
    parts = sum(OM.loss(params, cfg, *_pack([t], t.numel())) for t in docs)
    torch.testing.assert_close(total, parts, rtol=ltol, atol=ltol)


def test_model_oracle_is_causal() -> None:
    """Changing the tokens after position t leaves the loss at position t unchanged,
    and changing the token at t changes it (the mask is causal, not bidirectional)."""
    from oracle import model as OM

    cfg, params = _tiny_model(seed=3)
    g = torch.Generator().manual_seed(1)
    toks = torch.randint(0, cfg.vocab_size, (12,), generator=g)
    ids, lab, pos, doc = _pack([toks], 12)
    t = 5
    only = torch.full_like(lab, -100)
    only[0, t] = lab[0, t]
    base = OM.loss(params, cfg, ids, only, pos, doc)
    later = ids.clone()
    later[0, t + 1:] = (later[0, t + 1:] + 3) % cfg.vocab_size
    torch.testing.assert_close(OM.loss(params, cfg, later, only, pos, doc), base,
                               rtol=1e-13, atol=1e-13)
    now = ids.clone()
    now[0, t] = (now[0, t] + 3) % cfg.vocab_size
    assert abs(float(OM.loss(params, cfg, now, only, pos, doc) - base)) > 1e-6


@pytest.mark.parametrize("z", [0.0, 0.05])
def test_model_oracle_zero_embeddings_give_log_vocab(z: float) -> None:
    """All-zero embeddings: every hidden state, norm output and logit is 0, so each
    labelled row costs ln V (+ z * (ln V)^2); ignored and pad rows cost nothing."""
    from oracle import model as OM

    cfg, params = _tiny_model(vocab=53, z=z)
    with torch.no_grad():
        params["embed_tokens.weight"].zero_()
    g = torch.Generator().manual_seed(2)
    docs = [torch.randint(0, cfg.vocab_size, (n,), generator=g) for n in (9, 3, 5)]
    ids, lab, pos, doc = _pack(docs, 21)
    n_valid = int((lab != -100).sum())
    assert n_valid == 9 + 3 + 5 - 3
    want = n_valid * (math.log(53) + z * math.log(53) ** 2)
    got = float(OM.loss(params, cfg, ids, lab, pos, doc).detach())
    # the z-loss lse is an fp32 logsumexp (reference.py:45)
    assert abs(got - want) < (1e-7 if z else 1e-12) * want


def test_model_oracle_rope_matches_pinned_rotation() -> None:
    """oracle/model.py's RoPE (fp32 frequency table, rope.py:9-18) against the
    invariant-pinned oracle.kernels.rope with angles p * theta^(-2i/D) computed
    independently in float64; tolerance from the fp32 angles (|p| < 64)."""
    from oracle import model as OM

    g = torch.Generator().manual_seed(4)
    B, H, Hk, S, D, base = 2, 3, 1, 9, 16, 10000.0
    q = torch.randn(B, H, S, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, Hk, S, D, generator=g, dtype=torch.float64)
    pos = torch.randint(0, 64, (B, S), generator=g)
    pos[0, 0] = 0
    ang = pos.numpy()[..., None].astype(np.float64) * base ** (-np.arange(0, D, 2) / D)
    c, s = torch.from_numpy(np.cos(ang)), torch.from_numpy(np.sin(ang))
    qo, ko = OM._rope(q, k, pos, D, base)
    torch.testing.assert_close(qo, OK.rope(q, c, s), rtol=0, atol=2e-5)
    torch.testing.assert_close(ko, OK.rope(k, c, s), rtol=0, atol=2e-5)
    # position 0 is the identity exactly
    torch.testing.assert_close(qo[0, :, 0], q[0, :, 0], rtol=0, atol=0)


def test_model_oracle_pins_catch_planted_mistakes(monkeypatch) -> None:
    """The packed-vs-isolated invariant fails for an attention that ignores the
    document ids.  (Absolute pack positions would pass it: RoPE scores depend only
    on q - k position differences inside a document; the RoPE table is pinned by
    test_model_oracle_rope_matches_pinned_rotation.)"""
    from oracle import model as OM

    cfg, params = _tiny_model(seed=5)
    g = torch.Generator().manual_seed(9)
    docs = [torch.randint(0, cfg.vocab_size, (n,), generator=g) for n in (5, 7)]
    ids, lab, pos, doc = _pack(docs, 12)
    only = torch.full_like(lab, -100)
    only[0, 5:12] = lab[0, 5:12]  # the second document
    alone = OM.loss(params, cfg, *_pack([docs[1]], 7))

    def differs(**kw) -> bool:
        args = dict(input_ids=ids, labels=only, position_ids=pos, doc_ids=doc) | kw
        got = OM.loss(params, cfg, args["input_ids"], args["labels"], args["position_ids"],
                      args["doc_ids"])
        return abs(float((got - alone).detach())) > 1e-6

    assert not differs()
    with monkeypatch.context() as m:
        m.setattr(OM, "_eager_attention",
                  lambda q, k, v, d: F.scaled_dot_product_attention(
                      q, k.repeat_interleave(q.shape[1] // k.shape[1], 1),
                      v.repeat_interleave(q.shape[1] // k.shape[1], 1), is_causal=True))
        assert differs()


# ---------------------------------------------------------------- model composition
def _np_rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def _np_ce_sum(h: np.ndarray, emb: np.ndarray, labels: np.ndarray) -> float:
    """Sum over labelled rows of logsumexp(h E^T) - (h E^T)[label], by hand."""
    z = h @ emb.T
    m = z.max(-1, keepdims=True)
    lse = (m + np.log(np.exp(z - m).sum(-1, keepdims=True)))[:, 0]
    rows = np.nonzero(labels != -100)[0]
    return float(sum(lse[t] - z[t, labels[t]] for t in rows))


def _one_layer(seed: int):
    cfg, params = _tiny_model(seed=seed)
    cfg.n_layers = 1
    params = {n: t for n, t in params.items() if not n.startswith("layers.1.")}
    # Logits ~4x larger than at init, so the summed CE resolves the direction
    # of the final hidden state (a composition mistake moves it by ~1e-2).
    with torch.no_grad():
        params["norm.weight"].mul_(4.0)
    return cfg, params


def _composition_case():
    g = torch.Generator().manual_seed(11)
    docs = [torch.randint(0, 37, (n,), generator=g) for n in (5, 1, 8)]
    return _pack(docs, 16)


def _attention_closed_form_error(loss_fn) -> float:
    """Relative loss error of `loss_fn` on a 1-layer model whose q/k projections
    are zero and whose MLP output is zero (down_proj = 0).

    Zero scores make each query's softmax uniform over its document's causal
    prefix, so head h's output at position t is the mean of the value rows
    (KV head h // G) over the positions tau <= t of t's document, and zero on
    pad rows.  With pre-norm residual blocks (llama.py:122-125):
        h1 = E[ids] + concat_h(prefix mean of v_h) Wo^T,  v = rmsnorm(E[ids]; w1) Wv^T
    then the final norm and the tied LM head give the summed CE."""
    cfg, params = _one_layer(seed=21)
    with torch.no_grad():
        for n in ("q_proj", "k_proj"):
            params[f"layers.0.self_attn.{n}.weight"].zero_()
        params["layers.0.mlp.down_proj.weight"].zero_()
    ids, lab, pos, doc = _composition_case()
    P = {n: t.detach().numpy() for n, t in params.items()}
    eps, hd, G = cfg.norm_eps, cfg.d_model // cfg.n_heads, cfg.n_heads // cfg.n_kv_heads
    h0 = P["embed_tokens.weight"][ids[0].numpy()]
    v = _np_rmsnorm(h0, P["layers.0.input_layernorm.weight"], eps) @ P["layers.0.self_attn.v_proj.weight"].T
    d = doc[0].numpy()
    S = h0.shape[0]
    a = np.zeros((S, cfg.n_heads * hd))
    for t in range(S):
        if d[t] < 0:
            continue
        prefix = [tau for tau in range(t + 1) if d[tau] == d[t]]
        for h in range(cfg.n_heads):
            kvh = h // G
            a[t, h * hd:(h + 1) * hd] = v[prefix, kvh * hd:(kvh + 1) * hd].mean(0)
    h1 = h0 + a @ P["layers.0.self_attn.o_proj.weight"].T
    hf = _np_rmsnorm(h1, P["norm.weight"], eps)
    want = _np_ce_sum(hf, P["embed_tokens.weight"], lab[0].numpy())
    got = float(loss_fn(params, cfg, ids, lab, pos, doc).detach())
    return abs(got - want) / abs(want)


def _mlp_closed_form_error(loss_fn) -> float:
    """Relative loss error of `loss_fn` on a 1-layer model whose attention
    output is zero (v_proj = 0) and whose gate projection is twice its up
    projection.  Then gate = 2u with u = rmsnorm(E[ids]; w2) Wu^T, and
    silu(gate) * up = 2u * sigmoid(2u) * u, so
        h2 = E[ids] + (2 u^2 sigmoid(2u)) Wd^T
    (swapping the roles of gate and up would give 2 u^2 sigmoid(u))."""
    cfg, params = _one_layer(seed=22)
    with torch.no_grad():
        params["layers.0.self_attn.v_proj.weight"].zero_()
        params["layers.0.mlp.gate_proj.weight"].copy_(2.0 * params["layers.0.mlp.up_proj.weight"])
    ids, lab, pos, doc = _composition_case()
    P = {n: t.detach().numpy() for n, t in params.items()}
    eps = cfg.norm_eps
    h0 = P["embed_tokens.weight"][ids[0].numpy()]
    u = _np_rmsnorm(h0, P["layers.0.post_attention_layernorm.weight"], eps) @ P["layers.0.mlp.up_proj.weight"].T
    act = 2.0 * u * u / (1.0 + np.exp(-2.0 * u))
    h2 = h0 + act @ P["layers.0.mlp.down_proj.weight"].T
    hf = _np_rmsnorm(h2, P["norm.weight"], eps)
    want = _np_ce_sum(hf, P["embed_tokens.weight"], lab[0].numpy())
    got = float(loss_fn(params, cfg, ids, lab, pos, doc).detach())
    return abs(got - want) / abs(want)


# oracle/model.py computes RMSNorm in fp32 (reference.py:10 takes x.float()).
_COMPOSITION_TOL = 2e-6


def test_model_oracle_composition_closed_forms() -> None:
    """oracle/model.py's layer composition against two hand-computed closed forms:
    uniform attention (zero q/k projections) through o_proj into the residual
    stream, and a SwiGLU whose gate is twice its up projection."""
    from oracle import model as OM

    assert _attention_closed_form_error(OM.loss) < _COMPOSITION_TOL
    assert _mlp_closed_form_error(OM.loss) < _COMPOSITION_TOL


def test_model_oracle_composition_catches_planted_mistakes(monkeypatch) -> None:
    """Each of three composition mistakes planted in the oracle moves one of the
    closed forms far outside its tolerance: gate and up swapped (llama.py:57-61),
    the residual taken after the norm, and o_proj skipped (llama.py:102-103,
    122-125)."""
    from oracle import model as OM

    def swapped_mlp(x, p, pre):
        gate = x @ p[pre + "mlp.gate_proj.weight"].t()
        up = x @ p[pre + "mlp.up_proj.weight"].t()
        return (F.silu(up) * gate) @ p[pre + "mlp.down_proj.weight"].t()

    def post_norm_residual(h, p, pre, cfg, position_ids, doc_ids):
        eps = cfg.norm_eps
        x = OM._rmsnorm(h, p[pre + "input_layernorm.weight"], eps)
        h = x + OM._attention(x, p, pre, cfg, position_ids, doc_ids)
        x = OM._rmsnorm(h, p[pre + "post_attention_layernorm.weight"], eps)
        return x + OM._mlp(x, p, pre)

    real_attention = OM._attention

    def no_o_proj(x, p, pre, cfg, position_ids, doc_ids):
        q = dict(p)
        q[pre + "self_attn.o_proj.weight"] = torch.eye(cfg.d_model, dtype=x.dtype)
        return real_attention(x, q, pre, cfg, position_ids, doc_ids)

    for name, fn, check in (("_mlp", swapped_mlp, _mlp_closed_form_error),
                            ("_layer", post_norm_residual, _attention_closed_form_error),
                            ("_attention", no_o_proj, _attention_closed_form_error)):
        with monkeypatch.context() as m:
            m.setattr(OM, name, fn)
            err = check(OM.loss)
        assert err > 100 * _COMPOSITION_TOL, (name, err)
