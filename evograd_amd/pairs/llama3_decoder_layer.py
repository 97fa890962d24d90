"""One Llama-3 decoder layer as one autograd pair on gfx950.

Replaces the reference's level-3 operator
(src/evograd/ops/level3/llama3_decoder_layer/__init__.py:136-235, forward
forward_ref.py:53-117):

    h1 = rmsnorm(x); q, k, v = h1 Wq^T, h1 Wk^T, h1 Wv^T; q, k rotated (RoPE)
    o = causal GQA attention(q, k, v); x1 = x + o Wo^T
    h2 = rmsnorm(x1); act = silu(h2 Wg^T) * (h2 Wu^T); out = x1 + act Wd^T

composed from this library's kernels, every step on the GPU through the C ABI:
``eg_rmsnorm_fwd/bwd`` for the norms; ``eg_gemm`` (MFMA for 16-bit operands) for
the seven projections and their gradients, the residual adds folded into the
epilogues of the products that feed them (``x1 = x + o Wo^T``, ``out = x1 + act
Wd^T``, and the sums ``dh = dq Wq + dk Wk + dv Wv``, ``dh2 = dgate Wg + dup Wu``);
``eg_split_heads`` / ``eg_merge_heads`` for the [B, T, H, D] <-> [B, H, T, D]
layout changes with the RoPE rotation (and, backward, its transpose) applied on
the way (``eg_split_qkv_heads`` / ``eg_merge_qkv_heads``: q, k and v of the fused
projection in one launch); ``eg_attn_gqa_fwd/bwd`` for the attention (MFMA at 16-bit head_dim 64 or
128, the generic kernels for the fp32 and head_dim 16/32 correctness cases);
``eg_silu_mul`` / ``eg_swiglu_bwd`` for the MLP activation; ``eg_add`` where the
residual gradient meets a norm's.

Saved state (the block-level choice the reference's note invites, :190-199): the
ten inputs and the tables (references, no new storage), the attention output ``o``
[B*T, q_out], its ``lse`` [B, H, T] fp32, the residual stream ``x1`` [B*T, hidden]
and the two norms' ``rstd`` [B*T] fp32. Everything else is recomputed in the
backward: h1 and h2 (norm passes), q/k/v (three products), gate and up (two
products) and the activation. At B=1, T=4096 with Llama-3-8B widths the new saved
storage is 67.6 MB (bf16) where keeping every intermediate would hold about 690 MB;
the price is 1.17 TFLOP of recomputed products (the q/k/v and gate/up projections).

16-bit operands need hidden % 64 == 0 (the products' k step). An intermediate size
that is not a multiple of 64 is handled by zero-padded activation rows (and a
zero-padded copy of Wd for the down projection, whose operands are both
k-contiguous); a kv width that is not, by zero-padded dk/dv rows.
"""

from __future__ import annotations

if not __package__:
    # Loaded from this file's path as a top-level candidate module (evograd's verify
    # and bench commands load a program that way): put the package root on sys.path.
    import pathlib as _pathlib
    import sys as _sys

    _ROOT = str(_pathlib.Path(__file__).resolve().parents[2])
    if _ROOT not in _sys.path:
        _sys.path.insert(0, _ROOT)

import ctypes
import math

import torch

from evograd_amd import _lib
from evograd_amd.pairs._util import as_contiguous, tag, workspace

_NAMES = ("x", "input_norm_weight", "q_weight", "k_weight", "v_weight", "o_weight",
          "post_norm_weight", "gate_weight", "up_weight", "down_weight")


def _pad64(n: int) -> int:
    return (n + 63) // 64 * 64


class _Shape:
    """The layer's widths, recovered from the tensors as the reference does
    (forward_ref.py:77-88): head counts from q_out // head_dim, kv_out // head_dim."""

    def __init__(self, x, wq, wk, wg, cos):
        self.B, self.T, self.hidden = x.shape
        self.M = self.B * self.T
        self.D = cos.shape[-1]
        self.q_out, self.kv_out, self.inter = wq.shape[0], wk.shape[0], wg.shape[0]
        if self.q_out % self.D or self.kv_out % self.D:
            raise ValueError("q_out and kv_out must be whole multiples of head_dim")
        self.H, self.KVH = self.q_out // self.D, self.kv_out // self.D
        if self.H % self.KVH:
            raise ValueError(f"GQA needs n_heads divisible by n_kv_heads, got {self.H} and "
                             f"{self.KVH}")
        wide = x.dtype != torch.float32
        # row strides: k-contiguous 16-bit operands of a product need k % 64 == 0
        self.Ip = _pad64(self.inter) if wide else self.inter
        self.kvp = _pad64(self.kv_out) if wide else self.kv_out
        # 16-bit widths in whole 256-wide tiles: the projections that share an input
        # (q, k, v; gate, up) run as one product over their concatenated weights
        self.qkv = self.q_out + 2 * self.kv_out
        self.fuse_qkv = wide and self.q_out % 256 == 0 and self.kv_out % 256 == 0
        self.fuse_mlp = wide and self.inter % 256 == 0
        # the input gradients as one product with the weights as segments along K, or
        # as separate products accumulating through the residual operand. q/k/v: one
        # product at every T (measured T = 1024 / 2048 / 4096: -51 / -59 / -69 us per
        # backward). gate/up: one product only while dh2 has at most 128 output tiles
        # (half the CUs), where the products split k and one split product beats two
        # (T = 1024: -17 us; at T = 4096, 256 tiles, one long product against two: +20 us)
        self.kseg_qkv = self.fuse_qkv
        self.kseg_mlp = self.fuse_mlp and (self.M + 255) // 256 * ((self.hidden + 255) // 256) <= 128
        if wide and self.hidden % 64:
            raise ValueError(f"llama3_decoder_layer: 16-bit inputs need hidden % 64 == 0, got "
                             f"{self.hidden}")


def _check(args):
    x, w_in, wq, wk, wv, wo, w_post, wg, wu, wd, cos, sin = args
    _lib.require_gpu("llama3_decoder_layer", *args)
    if x.dim() != 3:
        raise ValueError(f"llama3_decoder_layer: x must be [B, T, hidden], got {tuple(x.shape)}")
    B, T, hidden = x.shape
    dt = x.dtype
    tag(dt)
    for name, t in zip(_NAMES[1:], args[1:10]):
        if t.dtype != dt:
            raise TypeError(f"llama3_decoder_layer: {name} is {t.dtype}, x is {dt}")
    D = cos.shape[-1] if cos.dim() == 2 else -1
    q_out, kv_out, inter = wq.shape[0], wk.shape[0], wg.shape[0]
    want = {"input_norm_weight": (hidden,), "q_weight": (q_out, hidden),
            "k_weight": (kv_out, hidden), "v_weight": (kv_out, hidden),
            "o_weight": (hidden, q_out), "post_norm_weight": (hidden,),
            "gate_weight": (inter, hidden), "up_weight": (inter, hidden),
            "down_weight": (hidden, inter)}
    for name, t in zip(_NAMES[1:], args[1:10]):
        if tuple(t.shape) != want[name]:
            raise ValueError(f"llama3_decoder_layer: {name} must be {want[name]}, got "
                             f"{tuple(t.shape)}")
    if tuple(cos.shape) != (T, D) or tuple(sin.shape) != (T, D) or D <= 0 or D % 2:
        raise ValueError(f"llama3_decoder_layer: cos and sin must be [T, head_dim] with an even "
                         f"head_dim, got {tuple(cos.shape)}, {tuple(sin.shape)}")
    if cos.dtype != sin.dtype or cos.dtype not in (torch.float32, dt):
        raise TypeError("llama3_decoder_layer: cos and sin must both be fp32 or x's dtype")


class _Ops:
    """Thin callers of the C entry points on one stream and dtype."""

    def __init__(self, like: torch.Tensor):
        self.dev = like.device
        self.dt = like.dtype
        self.tg = tag(like.dtype)
        self.st = _lib.stream_of(like)

    def empty(self, *shape, dtype=None):
        return torch.empty(shape, dtype=dtype or self.dt, device=self.dev)

    def padded(self, rows, cols, ld):
        """[rows, ld] with the columns past cols zeroed (rows of a k-padded operand)."""
        if ld == cols:
            return self.empty(rows, ld)
        t = self.empty(rows, ld)
        t[:, cols:].zero_()
        return t

    def gemm(self, a, b, c, m, n, k, lda, ldb, ldc, akc, bkc, r=None, ldr=0):
        # products of few output tiles split k over a workspace (fp32 partials)
        nbytes = _lib.query("eg_gemm_workspace_bytes", m, n, k, self.tg)
        ws = workspace(nbytes, self.dev) if nbytes else None
        _lib.call("eg_gemm", _lib.ptr(a), _lib.ptr(b), _lib.ptr(c), _lib.ptr(r), m, n, k, lda,
                  ldb, ldc, ldr, int(akc), int(bkc), self.tg, self.tg, _lib.ptr(ws), nbytes,
                  self.st)

    def gemm_seg(self, a, b, c, m, n, k, lda, ldb, ldc, akc, bkc, dim, sizes, a_segs=None,
                 b_segs=None, c_segs=None):
        """eg_gemm_segmented: operands concatenated from separate buffers along dim
        (1 = M, 2 = N, 3 = K), segment extents `sizes`."""
        nbytes = _lib.query("eg_gemm_workspace_bytes", m, n, k, self.tg)
        ws = workspace(nbytes, self.dev) if nbytes else None
        n_seg = len(sizes)
        arr = lambda ts: (ctypes.c_void_p * n_seg)(*[t.data_ptr() for t in ts]) if ts else None
        _lib.call("eg_gemm_segmented", _lib.ptr(a), _lib.ptr(b), _lib.ptr(c), m, n, k, lda, ldb,
                  ldc, int(akc), int(bkc), dim, n_seg, (ctypes.c_int64 * n_seg)(*sizes),
                  arr(a_segs), arr(b_segs), arr(c_segs), self.tg, self.tg, _lib.ptr(ws), nbytes,
                  self.st)

    def linear(self, h, w, out, m, n, k, ldh, ldo, r=None):
        """out[m, :n] = r + h[m, :k] w^T, w [n, k] (F.linear)."""
        self.gemm(h, w, out, m, n, k, ldh, w.shape[1], ldo, True, True, r, ldo if r is not None
                  else 0)

    def linear_dinput(self, dy, w, out, m, n, k, ldy, ldo, r=None):
        """out[m, :k] = r + dy[m, :n] w, w [n, k] (gradient of F.linear's input); n is the
        product's depth, padded in dy's row stride."""
        self.gemm(dy, w, out, m, k, n, ldy, w.shape[1], ldo, True, False, r,
                  ldo if r is not None else 0)

    def linear_dweight(self, dy, h, dw, m, n, k, ldy, ldh):
        """dw[n, k] = dy[:m, :n]^T h[:m, :k] (gradient of F.linear's weight, summed
        over the m tokens in fp32)."""
        self.gemm(dy, h, dw, n, k, m, ldy, ldh, k, False, False)

    def rmsnorm_fwd(self, x, w, y, rstd, rows, eps):
        _lib.call("eg_rmsnorm_fwd", _lib.ptr(x), _lib.ptr(w), _lib.ptr(y), _lib.ptr(rstd), rows,
                  w.shape[0], float(eps), self.tg, self.st)

    def rmsnorm_bwd(self, dy, x, w, rstd, dx, dw, rows):
        hidden = w.shape[0]
        ws = workspace(_lib.query("eg_rmsnorm_workspace_bytes", rows, hidden), self.dev)
        _lib.call("eg_rmsnorm_bwd", _lib.ptr(dy), _lib.ptr(x), _lib.ptr(w), _lib.ptr(rstd),
                  _lib.ptr(dx), _lib.ptr(dw), _lib.ptr(ws), rows, hidden, self.tg, self.st)

    def split(self, src, dst, s, heads, ld, rope, cos=None, sin=None):
        _lib.call("eg_split_heads", _lib.ptr(src), _lib.ptr(dst), _lib.ptr(cos), _lib.ptr(sin),
                  s.B, s.T, heads, s.D, ld, rope, tag(cos.dtype) if cos is not None else self.tg,
                  self.tg, self.st)

    def merge(self, src, dst, s, heads, ld, rope, cos=None, sin=None):
        _lib.call("eg_merge_heads", _lib.ptr(src), _lib.ptr(dst), _lib.ptr(cos), _lib.ptr(sin),
                  s.B, s.T, heads, s.D, ld, rope, tag(cos.dtype) if cos is not None else self.tg,
                  self.tg, self.st)

    def split_qkv(self, qkv, qh, kh, vh, s, cos, sin):
        """The rotated q, k and the copied v heads of the fused [q | k | v] rows, one
        launch."""
        _lib.call("eg_split_qkv_heads", _lib.ptr(qkv), _lib.ptr(qh), _lib.ptr(kh), _lib.ptr(vh),
                  _lib.ptr(cos), _lib.ptr(sin), s.B, s.T, s.H, s.KVH, s.D, s.qkv, 1,
                  tag(cos.dtype), self.tg, self.st)

    def merge_qkv(self, dqh, dkh, dvh, dqkv, s, cos, sin):
        """dq, dk (transpose-rotated) and dv into the fused [dq | dk | dv] rows, one
        launch."""
        _lib.call("eg_merge_qkv_heads", _lib.ptr(dqh), _lib.ptr(dkh), _lib.ptr(dvh),
                  _lib.ptr(dqkv), _lib.ptr(cos), _lib.ptr(sin), s.B, s.T, s.H, s.KVH, s.D, s.qkv,
                  2, tag(cos.dtype), self.tg, self.st)

    def add(self, a, b, c):
        _lib.call("eg_add", _lib.ptr(a), _lib.ptr(b), _lib.ptr(c), c.numel(), self.tg, self.st)


def _qkv_heads(ops, s, h1, wq, wk, wv, cos, sin):
    """q, k, v projections of h1, rotated (q, k) and split into [B, heads, T, D]. With
    the widths whole tiles, one product [q | k | v] = h1 [Wq; Wk; Wv]^T (the weights
    as segments along N) into one [M, q_out + 2 kv_out] buffer."""
    qh = ops.empty(s.B, s.H, s.T, s.D)
    kh = ops.empty(s.B, s.KVH, s.T, s.D)
    vh = ops.empty(s.B, s.KVH, s.T, s.D)
    if s.fuse_qkv:
        qkv = ops.empty(s.M, s.qkv)
        ops.gemm_seg(h1, None, qkv, s.M, s.qkv, s.hidden, s.hidden, s.hidden, s.qkv, True, True,
                     2, [s.q_out, s.kv_out, s.kv_out], b_segs=[wq, wk, wv])
        ops.split_qkv(qkv, qh, kh, vh, s, cos, sin)
        return qh, kh, vh
    q = ops.empty(s.M, s.q_out)
    k = ops.empty(s.M, s.kv_out)
    v = ops.empty(s.M, s.kv_out)
    ops.linear(h1, wq, q, s.M, s.q_out, s.hidden, s.hidden, s.q_out)
    ops.linear(h1, wk, k, s.M, s.kv_out, s.hidden, s.hidden, s.kv_out)
    ops.linear(h1, wv, v, s.M, s.kv_out, s.hidden, s.hidden, s.kv_out)
    ops.split(q, qh, s, s.H, s.q_out, 1, cos, sin)
    ops.split(k, kh, s, s.KVH, s.kv_out, 1, cos, sin)
    ops.split(v, vh, s, s.KVH, s.kv_out, 0)
    return qh, kh, vh


def _mlp_in(ops, s, h2, wg, wu):
    """gate, up = h2 Wg^T, h2 Wu^T as [M, Ip] rows (padding columns zero). With whole
    tiles, one product with [Wg; Wu] as segments along N and the two outputs as the
    segments of C: gate and up are the two halves of one [2, M, Ip] buffer."""
    if s.fuse_mlp:
        gu = ops.empty(2, s.M, s.Ip)
        ops.gemm_seg(h2, None, None, s.M, 2 * s.inter, s.hidden, s.hidden, s.hidden, s.Ip, True,
                     True, 2, [s.inter, s.inter], b_segs=[wg, wu], c_segs=[gu[0], gu[1]])
        return gu[0], gu[1]
    gate = ops.padded(s.M, s.inter, s.Ip)
    up = ops.padded(s.M, s.inter, s.Ip)
    ops.linear(h2, wg, gate, s.M, s.inter, s.hidden, s.hidden, s.Ip)
    ops.linear(h2, wu, up, s.M, s.inter, s.hidden, s.hidden, s.Ip)
    return gate, up


def _silu_mul(ops, gate, up):
    act = ops.empty(*gate.shape)
    _lib.call("eg_silu_mul", _lib.ptr(gate), _lib.ptr(up), _lib.ptr(act), act.numel(), ops.tg,
              ops.st)
    return act


def _down_weight_k_padded(ops, s, wd):
    """Wd [hidden, inter] as the k-contiguous operand of act Wd^T: rows padded to Ip."""
    if s.Ip == s.inter:
        return wd
    w = torch.zeros((s.hidden, s.Ip), dtype=wd.dtype, device=wd.device)
    w[:, :s.inter] = wd
    return w


def llama3_decoder_layer_forward_with_saved(x, input_norm_weight, q_weight, k_weight, v_weight,
                                            o_weight, post_norm_weight, gate_weight, up_weight,
                                            down_weight, cos, sin, eps: float = 1e-5):
    args = [x, input_norm_weight, q_weight, k_weight, v_weight, o_weight, post_norm_weight,
            gate_weight, up_weight, down_weight, cos, sin]
    _check(args)
    (x, w_in, wq, wk, wv, wo, w_post, wg, wu, wd, cos, sin) = [
        as_contiguous(n, t) for n, t in zip(_NAMES + ("cos", "sin"), args)]
    s = _Shape(x, wq, wk, wg, cos)
    ops = _Ops(x)
    x2 = x.view(s.M, s.hidden)
    h1 = ops.empty(s.M, s.hidden)
    rstd1 = ops.empty(s.M, dtype=torch.float32)
    ops.rmsnorm_fwd(x2, w_in, h1, rstd1, s.M, eps)
    qh, kh, vh = _qkv_heads(ops, s, h1, wq, wk, wv, cos, sin)
    del h1
    oh = ops.empty(s.B, s.H, s.T, s.D)
    lse = ops.empty(s.B, s.H, s.T, dtype=torch.float32)
    _lib.call("eg_attn_gqa_fwd", _lib.ptr(qh), _lib.ptr(kh), _lib.ptr(vh), _lib.ptr(oh),
              _lib.ptr(lse), s.B, s.H, s.KVH, s.T, s.D, 1.0 / math.sqrt(s.D), ops.tg, ops.st)
    del qh, kh, vh
    o = ops.empty(s.M, s.q_out)
    ops.merge(oh, o, s, s.H, s.q_out, 0)
    del oh
    x1 = ops.empty(s.M, s.hidden)
    ops.linear(o, wo, x1, s.M, s.hidden, s.q_out, s.q_out, s.hidden, r=x2)  # x + o Wo^T
    h2 = ops.empty(s.M, s.hidden)
    rstd2 = ops.empty(s.M, dtype=torch.float32)
    ops.rmsnorm_fwd(x1, w_post, h2, rstd2, s.M, eps)
    gate, up = _mlp_in(ops, s, h2, wg, wu)
    del h2
    act = _silu_mul(ops, gate, up)
    del gate, up
    out = ops.empty(s.M, s.hidden)
    ops.linear(act, _down_weight_k_padded(ops, s, wd), out, s.M, s.hidden, s.Ip, s.Ip, s.hidden,
               r=x1)  # x1 + act Wd^T
    saved = (x, w_in, wq, wk, wv, wo, w_post, wg, wu, wd, cos, sin, rstd1, o, lse, x1, rstd2)
    return out.view(s.B, s.T, s.hidden), saved


def llama3_decoder_layer_backward_from_saved(dout, saved, eps: float = 1e-5):
    x, w_in, wq, wk, wv, wo, w_post, wg, wu, wd, cos, sin, rstd1, o, lse, x1, rstd2 = saved
    _lib.require_gpu("llama3_decoder_layer_backward_from_saved", dout, x, o, x1)
    if dout.shape != x.shape or dout.dtype != x.dtype:
        raise ValueError("llama3_decoder_layer: dout must match x in shape and dtype")
    dout = as_contiguous("dout", dout)
    s = _Shape(x, wq, wk, wg, cos)
    ops = _Ops(x)
    M, hidden = s.M, s.hidden
    x2 = x.view(M, hidden)
    dout2 = dout.view(M, hidden)

    # ---- MLP: recompute h2, gate, up and the activation
    h2 = ops.empty(M, hidden)
    ops.rmsnorm_fwd(x1, w_post, h2, ops.empty(M, dtype=torch.float32), M, eps)
    gate, up = _mlp_in(ops, s, h2, wg, wu)
    act = _silu_mul(ops, gate, up)
    # out = x1 + act Wd^T
    d_act = ops.padded(M, s.inter, s.Ip)
    ops.linear_dinput(dout2, wd, d_act, M, hidden, s.inter, hidden, s.Ip)
    d_wd = ops.empty(hidden, s.inter)
    ops.linear_dweight(dout2, act, d_wd, M, hidden, s.inter, hidden, s.Ip)
    del act
    # act = silu(gate) * up: dgate, dup in place of gate, up (read before written)
    _lib.call("eg_swiglu_bwd", _lib.ptr(d_act), _lib.ptr(gate), _lib.ptr(up), _lib.ptr(gate),
              _lib.ptr(up), gate.numel(), ops.tg, ops.st)
    dgate, dup = gate, up
    del d_act
    dh2 = ops.empty(M, hidden)
    if s.fuse_mlp:
        # dh2 = [dgate | dup] [Wg; Wu] (segments along K); [dWg; dWu] = [dgate | dup]^T h2
        # (A's columns in two segments along M) into one buffer, returned as two views
        if s.kseg_mlp:
            ops.gemm_seg(None, None, dh2, M, hidden, 2 * s.inter, s.Ip, hidden, hidden, True,
                         False, 3, [s.inter, s.inter], a_segs=[dgate, dup], b_segs=[wg, wu])
        else:
            ops.linear_dinput(dgate, wg, dh2, M, s.inter, hidden, s.Ip, hidden)
            ops.linear_dinput(dup, wu, dh2, M, s.inter, hidden, s.Ip, hidden, r=dh2)
        d_wgu = ops.empty(2 * s.inter, hidden)
        ops.gemm_seg(None, h2, d_wgu, 2 * s.inter, hidden, M, s.Ip, hidden, hidden, False, False,
                     1, [s.inter, s.inter], a_segs=[dgate, dup])
        d_wg, d_wu = d_wgu[:s.inter], d_wgu[s.inter:]
    else:
        ops.linear_dinput(dgate, wg, dh2, M, s.inter, hidden, s.Ip, hidden)
        ops.linear_dinput(dup, wu, dh2, M, s.inter, hidden, s.Ip, hidden, r=dh2)
        d_wg = ops.empty(s.inter, hidden)
        d_wu = ops.empty(s.inter, hidden)
        ops.linear_dweight(dgate, h2, d_wg, M, s.inter, hidden, s.Ip, hidden)
        ops.linear_dweight(dup, h2, d_wu, M, s.inter, hidden, s.Ip, hidden)
    del dgate, dup, gate, up, h2
    # h2 = rmsnorm(x1); dx1 = dout (residual) + the norm's input gradient
    dx1 = ops.empty(M, hidden)
    d_wpost = torch.empty_like(w_post)
    ops.rmsnorm_bwd(dh2, x1, w_post, rstd2, dx1, d_wpost, M)
    ops.add(dx1, dout2, dx1)
    del dh2

    # ---- attention block: x1 = x + o Wo^T
    do_ = ops.empty(M, s.q_out)
    ops.linear_dinput(dx1, wo, do_, M, hidden, s.q_out, hidden, s.q_out)
    d_wo = ops.empty(hidden, s.q_out)
    ops.linear_dweight(dx1, o, d_wo, M, hidden, s.q_out, hidden, s.q_out)
    # recompute h1 and the rotated q, k and v
    h1 = ops.empty(M, hidden)
    ops.rmsnorm_fwd(x2, w_in, h1, ops.empty(M, dtype=torch.float32), M, eps)
    qh, kh, vh = _qkv_heads(ops, s, h1, wq, wk, wv, cos, sin)
    oh = ops.empty(s.B, s.H, s.T, s.D)
    ops.split(o, oh, s, s.H, s.q_out, 0)
    doh = ops.empty(s.B, s.H, s.T, s.D)
    ops.split(do_, doh, s, s.H, s.q_out, 0)
    del do_
    dqh, dkh, dvh = torch.empty_like(qh), torch.empty_like(kh), torch.empty_like(vh)
    ws = workspace(_lib.query("eg_attn_gqa_workspace_bytes", s.B, s.H, s.KVH, s.T, s.D), x.device)
    _lib.call("eg_attn_gqa_bwd", _lib.ptr(doh), _lib.ptr(qh), _lib.ptr(kh), _lib.ptr(vh),
              _lib.ptr(oh), _lib.ptr(lse), _lib.ptr(dqh), _lib.ptr(dkh), _lib.ptr(dvh),
              _lib.ptr(ws), s.B, s.H, s.KVH, s.T, s.D, 1.0 / math.sqrt(s.D), ops.tg, ops.st)
    del qh, kh, vh, oh, doh, ws
    # back to token rows; the rotation's transpose takes dq, dk to the pre-rotation q, k
    dh1 = ops.empty(M, hidden)
    if s.fuse_qkv:
        # [dq | dk | dv] in one [M, q_out + 2 kv_out] buffer; dh1 = [dq | dk | dv] [Wq; Wk;
        # Wv] (the weights as segments along K); [dWq; dWk; dWv] = [dq | dk | dv]^T h1 in
        # one buffer, returned as three views
        dqkv = ops.empty(M, s.qkv)
        ops.merge_qkv(dqh, dkh, dvh, dqkv, s, cos, sin)
        del dqh, dkh, dvh
        if s.kseg_qkv:
            ops.gemm_seg(dqkv, None, dh1, M, hidden, s.qkv, s.qkv, hidden, hidden, True, False,
                         3, [s.q_out, s.kv_out, s.kv_out], b_segs=[wq, wk, wv])
        else:
            ops.linear_dinput(dqkv, wq, dh1, M, s.q_out, hidden, s.qkv, hidden)
            ops.linear_dinput(dqkv[:, s.q_out:], wk, dh1, M, s.kv_out, hidden, s.qkv, hidden,
                              r=dh1)
            ops.linear_dinput(dqkv[:, s.q_out + s.kv_out:], wv, dh1, M, s.kv_out, hidden, s.qkv,
                              hidden, r=dh1)
        d_wqkv = ops.empty(s.qkv, hidden)
        ops.linear_dweight(dqkv, h1, d_wqkv, M, s.qkv, hidden, s.qkv, hidden)
        d_wq = d_wqkv[:s.q_out]
        d_wk = d_wqkv[s.q_out:s.q_out + s.kv_out]
        d_wv = d_wqkv[s.q_out + s.kv_out:]
        del dqkv, h1
    else:
        dq = ops.empty(M, s.q_out)
        dk = ops.padded(M, s.kv_out, s.kvp)
        dv = ops.padded(M, s.kv_out, s.kvp)
        ops.merge(dqh, dq, s, s.H, s.q_out, 2, cos, sin)
        ops.merge(dkh, dk, s, s.KVH, s.kvp, 2, cos, sin)
        ops.merge(dvh, dv, s, s.KVH, s.kvp, 0)
        del dqh, dkh, dvh
        ops.linear_dinput(dq, wq, dh1, M, s.q_out, hidden, s.q_out, hidden)
        ops.linear_dinput(dk, wk, dh1, M, s.kv_out, hidden, s.kvp, hidden, r=dh1)
        ops.linear_dinput(dv, wv, dh1, M, s.kv_out, hidden, s.kvp, hidden, r=dh1)
        d_wq = ops.empty(s.q_out, hidden)
        d_wk = ops.empty(s.kv_out, hidden)
        d_wv = ops.empty(s.kv_out, hidden)
        ops.linear_dweight(dq, h1, d_wq, M, s.q_out, hidden, s.q_out, hidden)
        ops.linear_dweight(dk, h1, d_wk, M, s.kv_out, hidden, s.kvp, hidden)
        ops.linear_dweight(dv, h1, d_wv, M, s.kv_out, hidden, s.kvp, hidden)
        del dq, dk, dv, h1
    # h1 = rmsnorm(x); dx = dx1 (residual) + the norm's input gradient
    dx = ops.empty(M, hidden)
    d_win = torch.empty_like(w_in)
    ops.rmsnorm_bwd(dh1, x2, w_in, rstd1, dx, d_win, M)
    ops.add(dx, dx1, dx)
    return (dx.view(s.B, s.T, hidden), d_win, d_wq, d_wk, d_wv, d_wo, d_wpost, d_wg, d_wu, d_wd)
