"""The C-ABI library builds, loads and exports exactly what include/evograd_hip.h
declares; the Python binding declares the same set. No kernel is launched."""

import ctypes
import os
import re

import pytest
import torch

from evograd_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "evograd_hip.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(eg_[a-z0-9_]+)\s*\(", text))


def test_header_and_binding_agree():
    syms = header_symbols()
    assert syms == set(_lib.SIGNATURES), syms ^ set(_lib.SIGNATURES)


def test_binding_arity_matches_header():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(name + r"\s*\(([^)]*)\)", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), (name, params, args)


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_library_loads_and_exports_every_symbol():
    lib = _lib.load()
    for name in header_symbols():
        assert hasattr(lib, name), name
    assert lib.eg_abi_version() == _lib.ABI_VERSION
    assert lib.eg_last_error() is not None
    # size queries are pure host arithmetic
    # partial rows: 512 per 512 threads of workgroup width (the widest case is the
    # 16-bit vector path's narrowest workgroup), at most one per row
    assert lib.eg_rmsnorm_workspace_bytes(16384, 4096) == 512 * 4096 * 4
    assert lib.eg_layernorm_workspace_bytes(16384, 4096) == 2 * 512 * 4096 * 4
    assert lib.eg_rmsnorm_workspace_bytes(16384, 64) == 4096 * 64 * 4
    assert lib.eg_layernorm_workspace_bytes(3, 64) == 2 * 3 * 64 * 4
    assert lib.eg_rmsnorm_workspace_bytes(0, 64) == 0
    assert lib.eg_cross_entropy_workspace_bytes(8192) == 8192 * 4


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_flce_scratch_grows_with_the_chunk_not_with_rows_times_vocab():
    """The fused linear cross entropy holds the dlogits of one row chunk at a time
    (fused_linear_cross_entropy/__init__.py: "dlogits must not be materialized in
    full"): at the Llama-3 lm_head size its scratch is one chunk of dlogits, one
    chunk of group statistics, 12 bytes per row and, over several chunks, the fp32
    dweight sum, whatever the row count."""
    vocab, hidden, bf16 = 128256, 4096, _lib.EG_BF16

    def al(n):
        return (n + 255) // 256 * 256

    def expect(rows, rc):
        nh2 = 2 * ((vocab + 255) // 256)
        acc = al(vocab * hidden * 4) if rows > rc else 0  # the fp32 dweight sum
        return al(rows * 8) + al(rows * 4) + al(rc * nh2 * 8) + al(rc * vocab * 2) + acc

    ws = lambda rows, rc: _lib.query("eg_flce_workspace_bytes", rows, hidden, vocab, rc, bf16)
    # default: as many rows as 1 GiB of dlogits allows, a multiple of 256 -> 4096
    assert ws(8192, 0) == expect(8192, 4096)
    assert ws(65536, 0) == expect(65536, 4096)
    assert ws(65536, 0) - ws(8192, 0) == al(65536 * 8) + al(65536 * 4) - al(8192 * 8) - al(8192 * 4)
    # one chunk of dlogits (at most 1 GiB) and a weight-sized fp32 sum, nothing rows x vocab
    assert ws(8192, 0) - al(vocab * hidden * 4) < 1.1 * (1 << 30)
    # an explicit chunk sets the size; it is capped by the rows
    assert ws(8192, 1024) == expect(8192, 1024)
    assert ws(8192, 2048) - ws(8192, 1024) == expect(8192, 2048) - expect(8192, 1024)
    assert ws(100, 4096) == expect(100, 100)
    # fp32 inputs: one chunk of fp32 logits and one of fp32 dlogits (2^28 each)
    f32 = _lib.query("eg_flce_workspace_bytes", 8192, hidden, vocab, 0, _lib.EG_F32)
    rc32 = (1 << 28) // vocab
    rc32 = 1 << (rc32.bit_length() - 1)
    assert f32 == al(8192 * 8) + 2 * al(rc32 * vocab * 4)


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_gemm_workspace_split_k_and_split_tail():
    """Split k (at most 128 tiles of 256 x 256): splits x M x N fp32. Split tail
    (more than 256 tiles, the last wave of 256 at most half full): parts x tail tiles
    of 256 x 256 fp32, parts = min(4, 256 / tail, slices / 4) rounded to whole slices."""
    q = lambda m, n, k: _lib.query("eg_gemm_workspace_bytes", m, n, k, _lib.EG_BF16)
    tile = 256 * 256 * 4
    assert q(1024, 1024, 4096) == 16 * 1024 * 1024 * 4        # 16 tiles: 16 splits
    assert q(4096, 4096, 4096) == 0                          # one full wave
    assert q(8192, 8192, 8192) == 0                          # 4 full waves
    assert q(4096, 14336, 4096) == 2 * 128 * tile            # 896 tiles: 128 in 2 parts
    assert q(14336, 4096, 4096) == 2 * 128 * tile
    assert q(2048, 14336, 4096) == 0                         # 448 tiles: last wave 3/4 full
    assert q(2048, 4096, 14336) == 2 * 2048 * 4096 * 4       # 128 tiles: 2 splits
    assert q(128256, 4096, 4096) == 3 * 80 * tile            # 8016 tiles: 80 in 3 parts
    assert q(4300, 4000, 704) == 2 * 16 * tile               # 272 tiles, 11 slices
    assert q(4300, 4000, 448) == 0                           # 7 slices: no two runs of 4
    assert _lib.query("eg_gemm_workspace_bytes", 4096, 14336, 4096, _lib.EG_F32) == 0


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_attention_workspace_holds_the_split_walk_only_when_split():
    """delta (fp32 [batch, heads, seq], rounded up to 256 bytes), plus the split dK/dV
    walk's fp32 slabs (2 x parts x batch x kv_heads x seq x head_dim) when fewer than
    1024 (kv head, 128-key block) pairs exist: parts = min(8, ceil(1024 / pairs))."""
    al = lambda n: (n + 255) // 256 * 256
    q = lambda *a: _lib.query("eg_attn_gqa_workspace_bytes", *a)
    assert q(4, 32, 8, 4096, 128) == al(4 * 32 * 4096 * 4)          # 1024 pairs: no split
    assert q(1, 32, 8, 4096, 128) == al(32 * 4096 * 4) + 2 * 4 * 8 * 4096 * 128 * 4
    assert q(1, 32, 8, 1024, 128) == al(32 * 1024 * 4) + 2 * 8 * 8 * 1024 * 128 * 4
    assert q(2, 8, 2, 300, 64) == al(2 * 8 * 300 * 4) + 2 * 8 * 4 * 300 * 64 * 4
    assert q(1, 4, 4, 64, 48) == al(4 * 64 * 4)                      # generic kernels
    assert _lib.query("eg_attn_workspace_bytes", 4, 32, 4096, 128) == al(4 * 32 * 4096 * 4)
    assert _lib.query("eg_attn_workspace_bytes", 1, 32, 4096, 128) == q(1, 32, 32, 4096, 128)
    lq = _lib.query("eg_llama3_attn_workspace_bytes", 1, 32, 8, 1024, 128)
    assert lq == 2 * (32 + 8) * 1024 * 128 + q(1, 32, 8, 1024, 128)


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_host_side_validation_errors_without_gpu():
    """Argument errors are reported before any launch (no device needed)."""
    with pytest.raises(RuntimeError, match="negative"):
        _lib.call("eg_softmax_fwd", None, None, -1, 4, _lib.EG_F32, None)
    with pytest.raises(RuntimeError, match="even"):
        _lib.call("eg_rope", None, None, None, None, None, None, 1, 1, 0, 4, 5, 0, 0, 0, None)
    with pytest.raises(RuntimeError, match="dtype"):
        _lib.call("eg_swiglu_fwd", 16, 16, 16, 8, 7, None)
    with pytest.raises(RuntimeError, match="zero classes"):
        _lib.call("eg_cross_entropy_fwd", 16, 16, 16, 16, 16, 16, 4, 0, -100, _lib.EG_F32, None)
    with pytest.raises(RuntimeError, match="null"):
        _lib.call("eg_cross_entropy_bwd", None, 16, 16, 16, 16, 16, 4, 8, -100, _lib.EG_F32,
                  None)
    with pytest.raises(RuntimeError, match="out of range"):
        _lib.call("eg_cross_entropy_bwd", 16, 16, 16, 16, 16, 16, (1 << 24) + 1, 8, -100,
                  _lib.EG_BF16, None)
    # the allocation-free backward refuses sizes whose partial rows exceed its scratch
    with pytest.raises(RuntimeError, match="more than the 16777216-byte scratch"):
        _lib.call("eg_rmsnorm_bwd_noalloc", 16, 16, 16, 16, 16, 16, 16384, 16384,
                  _lib.EG_BF16, None)
    with pytest.raises(RuntimeError, match="null"):
        _lib.call("eg_probe_mfma_bf16", None, None, 256, 1, None)
    with pytest.raises(RuntimeError, match="workgroups"):
        _lib.call("eg_probe_mfma_bf16", 16, 16, 0, 1, None)
    with pytest.raises(RuntimeError, match="kind must be"):
        _lib.call("eg_probe_mfma_mix", 4, 16, 16, 256, 1, None)
    with pytest.raises(RuntimeError, match="workgroups"):
        _lib.call("eg_probe_mfma_mix", 1, 16, 16, 0, 1, None)
    # empty inputs are a no-op, not an error
    _lib.call("eg_softmax_fwd", None, None, 0, 0, _lib.EG_F32, None)
    _lib.call("eg_cross_entropy_bwd", None, None, None, None, None, None, 0, 8, -100,
              _lib.EG_F32, None)


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_gemm_segmented_refuses_bad_segments_on_the_host():
    """Segment checks run on the host before any launch (no device needed)."""
    p = 1 << 20  # never dereferenced: the checks run before any launch
    segs = (ctypes.c_void_p * 2)(p, p)
    def call(dim, sizes, m, n, k, a_segs=None, b_segs=segs, c_segs=None):
        return _lib.call("eg_gemm_segmented", p, p, p, m, n, k, 1024, 1024, 1024, 1, 1, dim,
                         len(sizes), (ctypes.c_int64 * len(sizes))(*sizes), a_segs, b_segs,
                         c_segs, _lib.EG_BF16, _lib.EG_BF16, None, 0, None)
    with pytest.raises(RuntimeError, match="multiples of 256"):
        call(2, [200, 56], 256, 256, 64)
    with pytest.raises(RuntimeError, match="add up"):
        call(2, [256, 256], 256, 600, 64)
    with pytest.raises(RuntimeError, match="does not index"):
        call(1, [256, 256], 512, 256, 64)          # B segments along M
    with pytest.raises(RuntimeError, match="seg_dim"):
        call(4, [256, 256], 256, 512, 64)


def test_pairs_refuse_cpu_tensors():
    from evograd_amd.pairs import rmsnorm, softmax

    with pytest.raises(RuntimeError, match="GPU"):
        softmax.softmax_forward_with_saved(torch.zeros(2, 4))
    with pytest.raises(RuntimeError, match="GPU"):
        rmsnorm.rmsnorm_forward_with_saved(torch.zeros(2, 4), torch.ones(4))
