"""The C-ABI library loads and exports every symbol include/*.h declares (CPU only)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

from packbalance_amd import _native as N

ROOT = Path(__file__).resolve().parents[1]


def _declared() -> set[str]:
    names: set[str] = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(pb_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_loads() -> None:
    assert N.available(), N._load_error
    assert N.lib().pb_abi_version() == N.ABI_VERSION


def test_every_declared_symbol_is_exported_and_bound() -> None:
    declared = _declared()
    assert {"pb_rmsnorm_fwd", "pb_swiglu_fwd", "pb_ce_rows", "pb_doc_block_tables"} <= declared
    lib = ctypes.CDLL(str(N.LIB_PATH))
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    unbound = sorted(declared - set(N.SIGNATURES))
    assert not unbound, f"declared but without a ctypes signature: {unbound}"
    extra = sorted(set(N.SIGNATURES) - declared)
    assert not extra, f"bound but not declared in include/: {extra}"


def test_status_and_error_message_without_gpu() -> None:
    # Argument validation runs on the host before any HIP call.
    lib = N.lib()
    rc = lib.pb_swiglu_fwd(None, None, None, 16, 99, None)
    assert rc == N.PB_EINVAL
    assert b"dtype" in lib.pb_last_error()
    rc = lib.pb_rmsnorm_fwd(None, 70000, 0, None, 0, None, 70000, None, 4, 70000, 1e-5, None)
    assert rc == N.PB_EUNSUPPORTED


def test_workspace_query_is_host_only() -> None:
    lib = N.lib()
    assert lib.pb_rmsnorm_bwd_workspace_bytes(0, 16) == 0
    assert lib.pb_rmsnorm_bwd_workspace_bytes(32768, 4096) > 0


def test_ce_rows_dl_rejects_bad_dtype_on_host() -> None:
    lib = N.lib()
    rc = lib.pb_ce_rows_dl(None, 8, 1, N.PB_F32, None, None, None, None, 8, 1, 99, 1, 8, -100,
                           0.0, None)
    assert rc == N.PB_EINVAL
    assert b"dlogits dtype" in lib.pb_last_error()


def test_vocab_chunk_budget() -> None:
    from packbalance_amd.kernels.fused_ce import CHUNK_BUDGET, VOCAB_CHUNK, vocab_chunk

    assert vocab_chunk(16384, 128256) == 32768  # cfg4: 4 chunks of dlogits
    assert vocab_chunk(4096, 32000) == 32000  # a cfg2 micro-batch: the whole vocabulary
    for n, v in [(1, 7), (129, 8200), (16384, 128256), (10**6, 50000), (37, 100003)]:
        c = vocab_chunk(n, v)
        v8 = (v + 7) // 8 * 8
        assert c % 8 == 0 and min(VOCAB_CHUNK, v8) <= c <= v8
        assert n * c <= max(CHUNK_BUDGET, n * VOCAB_CHUNK)


def test_ce_dlogits_rejects_bad_chunks_on_host() -> None:
    """pb_lmhead_ce_dlogits validates the vocab chunk and the strides before any launch."""
    lib = N.lib()
    args = lambda v0, vc, ldl, lg_dtype: (  # noqa: E731
        16, 8, 16, 8, 8, 64, 8, 16, -100, 0.0, 16, 16, v0, vc, 16, ldl, 16, 8, lg_dtype, None, 0,
        None)
    assert lib.pb_lmhead_ce_dlogits(*args(60, 8, 8, N.PB_BF16)) == N.PB_EINVAL  # past v
    assert b"chunk" in lib.pb_last_error()
    assert lib.pb_lmhead_ce_dlogits(*args(0, 16, 8, N.PB_BF16)) == N.PB_EINVAL  # ldl < vc
    assert lib.pb_lmhead_ce_dlogits(*args(0, 8, 8, 99)) == N.PB_EINVAL  # logits dtype


def test_ce_backward_split_k_choice_on_host() -> None:
    """The dx product's split-K count, read back from the backward workspace size
    (dL, dL^T, the fp32 dx accumulator, then one fp32 [n, d] partial per split):
    a grid of 96 256x128 tiles (a cfg2 micro-batch) takes 8 splits, three full
    rounds of 256 workgroups; cfg4's 2048 tiles take none."""
    lib = N.lib()

    def al(x):
        return (x + 255) // 256 * 256

    def splits(n, v, d, vchunk):
        base = al(n * vchunk * 2) + al(vchunk * ((n + 7) // 8 * 8) * 2) + al(n * d * 4)
        extra = lib.pb_lmhead_ce_bwd_workspace_bytes(n, v, d, vchunk) - base
        return 1 if extra == 0 else extra // (n * d * 4)

    assert splits(4096, 32000, 768, 32000) == 8
    assert splits(16384, 128256, 4096, 8192) == 1
    assert splits(512, 512, 128, 512) == 1  # a 512-column chunk cannot be split


def test_attention_kept_ds_config_on_host() -> None:
    """pb_attn_config: head dim 128 on a full grid with G % 4 == 0 keeps dS (64-row
    dQ tiles; workspace = delta + one G * 8 KiB block per causal 64 x 64 tile and
    (pack, KV head)); other shapes keep the recompute backward."""
    from packbalance_amd.model.attention import attn_config

    def ws_ds(b, hq, hkv, s):
        tri = (s // 64) * (s // 64 + 1) // 2
        return (b * hq * s * 4 + 255) // 256 * 256 + b * hkv * tri * (hq // hkv) * 8192

    c = attn_config(8, 32, 8, 8192, 128)  # cfg3
    assert c["tiles"][2] == (64, 64) and c["workspace"] == ws_ds(8, 32, 8, 8192)
    c = attn_config(8, 16, 2, 4096, 128)  # G = 8: two quads per KV head
    assert c["tiles"][2] == (64, 64) and c["workspace"] == ws_ds(8, 16, 2, 4096)
    for shape in [(2, 12, 4, 2048, 64),      # cfg2 micro-batch: D 64, G 3
                  (1, 8, 2, 1024, 128)]:     # small grid (split dK/dV partials)
        assert attn_config(*shape)["workspace"] != ws_ds(*shape[:4]), shape
    for shape in [(8, 24, 8, 8192, 128),     # G = 3
                  (8, 32, 8, 16384, 128)]:   # dS blocks beyond the 32 GiB cap
        c = attn_config(*shape)
        assert c["tiles"][2] == (128, 64) and c["workspace"] == (8 * shape[1] * shape[3] * 4), shape

