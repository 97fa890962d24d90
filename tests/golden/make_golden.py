"""Write the golden fixtures: tiny cases of every operator, computed in fp64 with
numpy alone (no torch, nothing from the reference).

Each ``<op>.npz`` holds the inputs (values exactly representable in bf16, so the
same case runs in fp32, fp16-free bf16 and fp32 paths), the upstream gradient,
the forward output, and every gradient. Forwards are written out from the
operators' definitions; gradients are central finite differences of
<dy, f(inputs)> in fp64 (step 1e-6, error ~1e-10), so no backward formula is
restated here. Run ``python tests/golden/make_golden.py`` to regenerate; the
fixtures are deterministic.
"""

from __future__ import annotations

import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_exact(a: np.ndarray) -> np.ndarray:
    """Round to the nearest bf16 value (ties to even), returned as fp64."""
    b = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return b.astype(np.uint32).view(np.float32).astype(np.float64)


def draw(rng, shape, scale=1.0):
    return bf16_exact(rng.standard_normal(shape) * scale)


# ------------------------------------------------------------------ forwards
def softmax(x):
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def rmsnorm(x, w, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def layernorm(x, w, b, eps):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def swiglu(a, b):
    return a / (1.0 + np.exp(-a)) * b


def rope_tables(tokens, dim, theta):
    inv = theta ** (-np.arange(0, dim, 2, dtype=np.float64) / dim)
    ang = np.arange(tokens, dtype=np.float64)[:, None] * inv[None, :]
    ang = np.concatenate([ang, ang], -1)
    return np.cos(ang), np.sin(ang)


def rope(x, cos, sin):
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], -1)
    return x * cos + rot * sin


def causal_attention(q, k, v):
    """q [B, H, S, D]; k, v [B, Hkv, S, D]; query head h reads kv head h // (H / Hkv)."""
    B, H, S, D = q.shape
    g = H // k.shape[1]
    out = np.zeros_like(q)
    for b in range(B):
        for h in range(H):
            kh, vh = k[b, h // g], v[b, h // g]
            for i in range(S):
                s = (kh[: i + 1] @ q[b, h, i]) / math.sqrt(D)
                p = np.exp(s - s.max())
                out[b, h, i] = (p / p.sum()) @ vh[: i + 1]
    return out


def cross_entropy(logits, target):
    tot, n = 0.0, 0
    for row, t in zip(logits, target):
        if t == -100:
            continue
        m = row.max()
        tot += m + math.log(np.exp(row - m).sum()) - row[t]
        n += 1
    return np.array(tot / n if n else float("nan"))


def flce(x, weight, target):
    return cross_entropy(x @ weight.T, target)


def decoder_layer(x, input_norm_weight, q_weight, k_weight, v_weight, o_weight,
                  post_norm_weight, gate_weight, up_weight, down_weight, cos, sin, eps=1e-5):
    """One Llama-3 decoder layer in fp64: x [B, T, hidden], weights [out, in]."""
    B, T, hid = x.shape
    D = cos.shape[-1]
    H, KVH = q_weight.shape[0] // D, k_weight.shape[0] // D

    def heads(lin, n):
        return lin.reshape(B, T, n, D).transpose(0, 2, 1, 3)

    h1 = rmsnorm(x, input_norm_weight, eps)
    q = rope(heads(h1 @ q_weight.T, H), cos, sin)
    k = rope(heads(h1 @ k_weight.T, KVH), cos, sin)
    v = heads(h1 @ v_weight.T, KVH)
    attn = causal_attention(q, k, v).transpose(0, 2, 1, 3).reshape(B, T, H * D)
    x1 = x + attn @ o_weight.T
    h2 = rmsnorm(x1, post_norm_weight, eps)
    return x1 + swiglu(h2 @ gate_weight.T, h2 @ up_weight.T) @ down_weight.T


# --------------------------------------------------------------- gradients
def fd_grads(f, inputs: dict, active, dy, h=1e-6):
    """d<dy, f>/d input for every Active input, by central differences."""
    grads = {}
    for name in active:
        base = inputs[name]
        g = np.zeros_like(base)
        flat = base.reshape(-1)
        gf = g.reshape(-1)
        for i in range(flat.size):
            keep = flat[i]
            step = h * max(1.0, abs(keep))
            flat[i] = keep + step
            hi = float((f(**inputs) * dy).sum())
            flat[i] = keep - step
            lo = float((f(**inputs) * dy).sum())
            flat[i] = keep
            gf[i] = (hi - lo) / (2 * step)
        grads["d" + name] = g
    return grads


def save(op, inputs, active, dy, f, scalars=None):
    out = f(**inputs)
    grads = fd_grads(f, inputs, active, dy)
    arrays = {f"in_{k}": v for k, v in inputs.items()}
    arrays.update({f"scalar_{k}": np.array(v) for k, v in (scalars or {}).items()})
    arrays["dy"] = dy
    arrays["out"] = out
    arrays.update({f"grad_{k}": v for k, v in grads.items()})
    np.savez(os.path.join(HERE, f"{op}.npz"), **arrays)
    print(f"{op}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in arrays.items()))


def main():
    rng = np.random.default_rng(20260601)
    x = draw(rng, (3, 8), 2.0)
    save("softmax", {"x": x}, ["x"], draw(rng, (3, 8)), softmax)

    eps = 1e-5
    x, w = draw(rng, (3, 16)), bf16_exact(1 + 0.1 * rng.standard_normal(16))
    save("rmsnorm", {"x": x, "weight": w}, ["x", "weight"], draw(rng, (3, 16)),
         lambda x, weight: rmsnorm(x, weight, eps), {"eps": eps})

    x, w, b = draw(rng, (3, 16)), draw(rng, (16,)), draw(rng, (16,))
    save("layernorm", {"x": x, "weight": w, "bias": b}, ["x", "weight", "bias"],
         draw(rng, (3, 16)), lambda x, weight, bias: layernorm(x, weight, bias, eps),
         {"eps": eps})

    a, bb = draw(rng, (4, 8), 2.0), draw(rng, (4, 8))
    save("swiglu", {"a": a, "b": bb}, ["a", "b"], draw(rng, (4, 8)), swiglu)

    cos, sin = rope_tables(4, 16, 10000.0)
    save("rope", {"x": draw(rng, (1, 2, 4, 16)), "cos": cos, "sin": sin}, ["x"],
         draw(rng, (1, 2, 4, 16)), rope)

    x, r, w = draw(rng, (3, 16)), draw(rng, (3, 16)), draw(rng, (16,))
    eps6 = 1e-6
    save("fused_add_rms_norm", {"x": x, "r": r, "weight": w}, ["x", "r", "weight"],
         draw(rng, (3, 16)), lambda x, r, weight: rmsnorm(x + r, weight, eps6), {"eps": eps6})

    qkv = {n: draw(rng, (1, 2, 5, 64)) for n in ("q", "k", "v")}
    save("causal_attention", qkv, ["q", "k", "v"], draw(rng, (1, 2, 5, 64)), causal_attention)

    gqa = {"q": draw(rng, (1, 4, 5, 64)), "k": draw(rng, (1, 2, 5, 64)),
           "v": draw(rng, (1, 2, 5, 64))}
    save("causal_attention_gqa", gqa, ["q", "k", "v"], draw(rng, (1, 4, 5, 64)), causal_attention)

    logits = draw(rng, (5, 12), 2.0)
    target = np.array([3, -100, 0, 11, 7], dtype=np.int64)
    save("cross_entropy", {"logits": logits, "target": target}, ["logits"],
         np.array(1.25), cross_entropy)

    xf, wf = draw(rng, (4, 8), 0.5), draw(rng, (12, 8), 8 ** -0.5)
    tf = np.array([2, 11, -100, 5], dtype=np.int64)
    save("fused_linear_cross_entropy", {"x": xf, "weight": wf, "target": tf}, ["x", "weight"],
         np.array(1.0), flce)

    # RoPE on q and k (exact fp64 rotation), then grouped causal attention
    cos, sin = rope_tables(5, 64, 10000.0)
    la = {"q": draw(rng, (1, 4, 5, 64)), "k": draw(rng, (1, 2, 5, 64)),
          "v": draw(rng, (1, 2, 5, 64)), "cos": cos, "sin": sin}
    save("llama3_attention", la, ["q", "k", "v"], draw(rng, (1, 4, 5, 64)),
         lambda q, k, v, cos, sin: causal_attention(rope(q, cos, sin), rope(k, cos, sin), v))

    # one decoder layer: B=1, T=3, hidden 8, head_dim 4, two query heads over one kv
    # head, intermediate 12; weights at fan-in scale, gains near 1
    hid, D, qo, kvo, inter, T = 8, 4, 8, 4, 12, 3
    cos, sin = rope_tables(T, D, 500000.0)
    layer = {
        "x": draw(rng, (1, T, hid), 0.5),
        "input_norm_weight": bf16_exact(1 + 0.1 * rng.standard_normal(hid)),
        "q_weight": draw(rng, (qo, hid), hid ** -0.5),
        "k_weight": draw(rng, (kvo, hid), hid ** -0.5),
        "v_weight": draw(rng, (kvo, hid), hid ** -0.5),
        "o_weight": draw(rng, (hid, qo), qo ** -0.5),
        "post_norm_weight": bf16_exact(1 + 0.1 * rng.standard_normal(hid)),
        "gate_weight": draw(rng, (inter, hid), hid ** -0.5),
        "up_weight": draw(rng, (inter, hid), hid ** -0.5),
        "down_weight": draw(rng, (hid, inter), inter ** -0.5),
        "cos": cos, "sin": sin,
    }
    save("llama3_decoder_layer", layer, [n for n in layer if n not in ("cos", "sin")],
         draw(rng, (1, T, hid), 0.5),
         lambda **kw: decoder_layer(**kw, eps=1e-5), {"eps": 1e-5})


if __name__ == "__main__":
    main()
