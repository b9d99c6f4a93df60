"""The benchmark graphs C1-C5 with their synthetic inputs.

Each builder draws its inputs from numpy PCG64 `default_rng(seed)` in a fixed
order, builds the graph with the reference's op semantics (tensor.py) and
returns (session, root tensor).  `scale` shrinks every dimension for tests
("small") while keeping the graph identical.

C1  MLP, fp32: logits = W2 relu(W1 x + b1) + b2 (nn.Linear layers, x @ W.T)
    x (64, 784) N(0,1); W1 (128, 784), b1 (128) ~ U(+-1/sqrt(784));
    W2 (10, 128), b2 (10) ~ U(+-1/sqrt(128))
C2  relu(a*b + c) * exp(-a*a) summed over axis 1; a, b, c (4096, 4096) N(0,1)
C3  x @ w + b; x, w (4096, 4096) U(-1, 1), b (4096,) U(-0.1, 0.1);
    fp32, or under autocast(float16)
C4  causal scaled_dot_product_attention, scale 0.125, Q K V (8, 16, 2048, 64)
    N(0,1) drawn in f32 then rounded to f16, under autocast(float16)
C5  one GPT-2 block under autocast(float16): x (8, 1024, 768) N(0,1);
    weights N(0, 0.02), biases 0, LayerNorm gamma 1 beta 0; 12 heads
"""
from __future__ import annotations

from typing import Optional, Tuple

import numpy as np

from .tensor import Session, Tensor, autocast, gelu, layer_norm, linear, relu, scaled_dot_product_attention


def _d(n: int, scale: float, mult: int = 1) -> int:
    return max(mult, int(round(n * scale / mult)) * mult)


def c1(scale: float = 1.0, seed: int = 1) -> Tuple[Session, Tensor]:
    rng = np.random.default_rng(seed)
    b, din, h, dout = _d(64, scale), _d(784, scale), _d(128, scale), 10
    s = Session()
    x = s.from_numpy(rng.standard_normal((b, din), dtype=np.float32), "x")
    bd1, bd2 = 1.0 / np.sqrt(din), 1.0 / np.sqrt(h)
    w1 = s.from_numpy(rng.uniform(-bd1, bd1, (h, din)).astype(np.float32), "W1")
    b1 = s.from_numpy(rng.uniform(-bd1, bd1, (h,)).astype(np.float32), "b1")
    w2 = s.from_numpy(rng.uniform(-bd2, bd2, (dout, h)).astype(np.float32), "W2")
    b2 = s.from_numpy(rng.uniform(-bd2, bd2, (dout,)).astype(np.float32), "b2")
    return s, linear(relu(linear(x, w1, b1)), w2, b2)


def c2(scale: float = 1.0, seed: int = 2) -> Tuple[Session, Tensor]:
    rng = np.random.default_rng(seed)
    n = _d(4096, scale)
    s = Session()
    a, b, c = (s.from_numpy(rng.standard_normal((n, n), dtype=np.float32), nm) for nm in "abc")
    y = relu(a * b + c) * ((-a) * a).exp()
    return s, y.sum(axis=1)


def c3(scale: float = 1.0, seed: int = 3, amp: bool = True) -> Tuple[Session, Tensor]:
    rng = np.random.default_rng(seed)
    n = _d(4096, scale, 16)
    s = Session()
    x = s.from_numpy(rng.uniform(-1, 1, (n, n)).astype(np.float32), "x")
    w = s.from_numpy(rng.uniform(-1, 1, (n, n)).astype(np.float32), "w")
    b = s.from_numpy(rng.uniform(-0.1, 0.1, (n,)).astype(np.float32), "b")
    with autocast("float16", enabled=amp):
        y = x @ w + b
    return s, y


def c4(scale: float = 1.0, seed: int = 4, dtype: str = "float16") -> Tuple[Session, Tensor]:
    rng = np.random.default_rng(seed)
    b, h, sq, d = _d(8, scale), _d(16, scale), _d(2048, scale), 64
    s = Session()
    q, k, v = (rng.standard_normal((b, h, sq, d), dtype=np.float32).astype(np.float16) for _ in range(3))
    tq, tk, tv = (s.from_numpy(t, nm) for t, nm in zip((q, k, v), "qkv"))
    with autocast(dtype):
        o = scaled_dot_product_attention(tq, tk, tv, is_causal=True, scale=0.125)
    return s, o


def gpt2_block(x: Tensor, p: dict, heads: int) -> Tensor:
    """Pre-LN GPT-2 block: x + proj(attn(ln1 x)); h + down(gelu(up(ln2 h)))."""
    bsz, seq, emb = x.shape
    hd = emb // heads
    h1 = layer_norm(x, emb, p["ln1_w"], p["ln1_b"])
    qkv = linear(h1, p["w_qkv"], p["b_qkv"])

    def heads_of(t: Tensor) -> Tensor:
        return t.reshape(bsz, seq, heads, hd).permute(0, 2, 1, 3)

    q = heads_of(qkv.slice(-1, 0, emb))
    k = heads_of(qkv.slice(-1, emb, 2 * emb))
    v = heads_of(qkv.slice(-1, 2 * emb, 3 * emb))
    a = scaled_dot_product_attention(q, k, v, is_causal=True)
    a = a.permute(0, 2, 1, 3).reshape(bsz, seq, emb)
    h = x + linear(a, p["w_o"], p["b_o"])
    h2 = layer_norm(h, emb, p["ln2_w"], p["ln2_b"])
    return h + linear(gelu(linear(h2, p["w_up"], p["b_up"])), p["w_down"], p["b_down"])


def c5(scale: float = 1.0, seed: int = 5, dtype: str = "float16",
       batch: Optional[int] = None) -> Tuple[Session, Tensor]:
    """C5; ``batch`` overrides the batch size alone (the CPU baseline times
    one sequence of the full-width block)."""
    rng = np.random.default_rng(seed)
    bsz, seq = _d(8, scale) if batch is None else batch, _d(1024, scale, 16)
    heads = 12 if scale >= 1.0 else 2
    emb = 768 if scale >= 1.0 else heads * 64
    s = Session()
    x = s.from_numpy(rng.standard_normal((bsz, seq, emb), dtype=np.float32), "x")

    def w(o: int, i: int, name: str) -> Tensor:
        return s.from_numpy((rng.standard_normal((o, i), dtype=np.float32) * np.float32(0.02)), name)

    def zeros(n: int, name: str) -> Tensor:
        return s.from_numpy(np.zeros((n,), dtype=np.float32), name)

    def ones(n: int, name: str) -> Tensor:
        return s.from_numpy(np.ones((n,), dtype=np.float32), name)

    p = {
        "w_qkv": w(3 * emb, emb, "w_qkv"), "w_o": w(emb, emb, "w_o"),
        "w_up": w(4 * emb, emb, "w_up"), "w_down": w(emb, 4 * emb, "w_down"),
        "b_qkv": zeros(3 * emb, "b_qkv"), "b_o": zeros(emb, "b_o"),
        "b_up": zeros(4 * emb, "b_up"), "b_down": zeros(emb, "b_down"),
        "ln1_w": ones(emb, "ln1_w"), "ln1_b": zeros(emb, "ln1_b"),
        "ln2_w": ones(emb, "ln2_w"), "ln2_b": zeros(emb, "ln2_b"),
    }
    with autocast(dtype):
        y = gpt2_block(x, p, heads)
    return s, y


BUILDERS = {"c1": c1, "c2": c2, "c3": c3, "c4": c4, "c5": c5}

__all__ = ["c1", "c2", "c3", "c4", "c5", "gpt2_block", "BUILDERS"]
