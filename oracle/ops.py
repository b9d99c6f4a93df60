"""Op-level NumPy restatements of the reference CPU realizer (test infrastructure).

Every function evaluates exactly what the reference's NumPy handlers compute
for one op (or one config-sized composite), in the same order of rounding
steps.  See oracle/__init__.py for how each one is pinned.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
F16 = np.float16

# ---------------------------------------------------------------------------
# dtype conversions
# ---------------------------------------------------------------------------


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """CAST f32 -> f16: NumPy astype, round to nearest even (_realize.py:210-212)."""
    return np.asarray(x, dtype=F32).astype(F16)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bfloat16 bit pattern (uint16).

    bfloat16 is not in the reference IR (_ir.py:348-353; _amp.py:123-128), so
    this restates the IEEE rule on the integer encoding: add 0x7fff plus the
    lsb of the kept half, truncate; NaNs stay quiet NaNs.
    """
    u = np.asarray(x, dtype=F32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """MATMUL handler (_realize.py:395-412): f16 operands are upcast, the
    product accumulates in f32 and the result is cast back to the node dtype
    (f16); f32 operands use a plain f32 ``a @ b``."""
    if a.dtype == F16 or b.dtype == F16:
        return (a.astype(F32) @ b.astype(F32)).astype(F16)
    return a @ b


def matmul_bf16(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """bf16 analogue of the AMP MATMUL (extension; no reference oracle):
    exact bf16 operands, f32 accumulation, result rounded to bf16 (bits)."""
    return f32_to_bf16_bits(bf16_bits_to_f32(a_bits) @ bf16_bits_to_f32(b_bits))


def linear_amp(x: np.ndarray, w: np.ndarray, b: np.ndarray | None) -> np.ndarray:
    """Autocast ``x @ w + b`` (C3-fp16): CAST x,w -> f16, MATMUL (f16 out),
    ADD promotes to f32 (_amp.py:56-69, 234-245)."""
    y = matmul(f32_to_f16(x), f32_to_f16(w))
    if b is not None:
        y = y.astype(F32) + b.astype(F32)
    return y


# ---------------------------------------------------------------------------
# Fused elementwise (_realize.py:1557-1600)
# ---------------------------------------------------------------------------

_NP_BINARY = {
    "ADD": np.add, "MUL": np.multiply, "DIV": np.divide, "SUB": np.subtract,
    "MAX": np.maximum, "MIN": np.minimum,
}
_NP_CMP = {
    "CMP_EQ": np.equal, "CMP_NE": np.not_equal, "CMP_LT": np.less,
    "CMP_LE": np.less_equal, "CMP_GT": np.greater, "CMP_GE": np.greater_equal,
}


def fused_program(inputs, ops, imms=()):
    """Evaluate an SSA op list the way ``_h_fused_elementwise`` does: refs < 0
    are inputs (-ref-1), refs >= 0 are earlier steps; every step is one NumPy
    ufunc call (so each op rounds to the array dtype).  Opcodes beyond the
    reference's six follow NumPy semantics in f32 (comparisons give 0/1)."""
    steps = []

    def res(r):
        return inputs[-r - 1] if r < 0 else steps[r]

    with np.errstate(all="ignore"):
        for op in ops:
            code, a = op[0], op[1]
            b = op[2] if len(op) > 2 else 0
            c = op[3] if len(op) > 3 else 0
            if code in _NP_BINARY:
                steps.append(_NP_BINARY[code](res(a), res(b)))
            elif code in _NP_CMP:
                steps.append(_NP_CMP[code](res(a), res(b)).astype(F32))
            elif code == "NEG":
                steps.append(-res(a))
            elif code == "EXP":
                steps.append(np.exp(res(a)))
            elif code == "LOG":
                steps.append(np.log(res(a)))
            elif code == "WHERE":
                steps.append(np.where(res(a) != 0, res(b), res(c)).astype(F32))
            elif code == "IMM":
                steps.append(F32(imms[a]))
            elif code == "ROUND_F16":
                steps.append(res(a).astype(F16).astype(F32))
            elif code == "ROUND_BF16":
                steps.append(round_bf16(res(a)))
            elif code == "TANH":
                steps.append(np.tanh(res(a)))
            elif code == "SQRT":
                steps.append(np.sqrt(res(a)))
            elif code == "RECIP":
                steps.append(F32(1.0) / res(a))
            elif code == "ABS":
                steps.append(np.abs(res(a)))
            elif code == "COPY":
                steps.append(res(a))
            else:
                raise ValueError(f"unknown opcode {code}")
    return steps[-1]


def c2_chain(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """C2: y = relu(a*b + c) * exp(-a*a); sum over axis 1.

    Graph order of the reference builders: MUL(a,b) -> ADD(c) ->
    relu = WHERE(CMP_gt(x, CONST 0), x, CONST 0) (_functional.py:99-112) ->
    NEG(a) -> MUL(neg, a) -> EXP -> MUL(relu, e) -> REDUCE sum axis=1
    (_realize.py:215-243, 386-393, 1094-1111, 1453-1459)."""
    with np.errstate(all="ignore"):
        t = a * b
        t = t + c
        zero = np.asarray(0.0, dtype=F32)
        r = np.where(t > zero, t, zero).astype(F32)
        e = np.exp((-a) * a)
        y = r * e
        return np.sum(y, axis=1)


# ---------------------------------------------------------------------------
# Normalisation / activations
# ---------------------------------------------------------------------------


def layer_norm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """LAYER_NORM handler (_realize.py:1008-1034), rows x cols in f32."""
    cols = x.shape[-1]
    x2 = x.reshape(-1, cols).astype(F32, copy=False)
    mean = x2.mean(axis=1, keepdims=True)
    centered = x2 - mean
    var = (centered * centered).mean(axis=1, keepdims=True)
    inv_std = 1.0 / np.sqrt(var + eps)
    x_hat = centered * inv_std
    out = x_hat * w.reshape(1, cols).astype(F32) + b.reshape(1, cols).astype(F32)
    return out.reshape(x.shape).astype(x.dtype, copy=False)


def _ln_rows(x: np.ndarray, cols: int, eps: float):
    """Row statistics shared by the LayerNorm handlers (_realize.py:1008-1023):
    f32 mean, centered values, biased variance, 1/sqrt(var + eps), x_hat."""
    x2 = np.asarray(x, dtype=F32).reshape(-1, cols)
    mean = x2.mean(axis=1, keepdims=True)
    centered = x2 - mean
    var = (centered * centered).mean(axis=1, keepdims=True)
    inv_std = F32(1.0) / np.sqrt(var + F32(eps))
    return inv_std, centered * inv_std


def layer_norm_backward_input(dy: np.ndarray, x: np.ndarray, w: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """LAYER_NORM_BACKWARD_INPUT handler (_realize.py:1036-1050):
    g = dy*w, dx = (inv_std/n) * ((n*g - sum(g)) - x_hat*sum(g*x_hat)), f32."""
    cols = x.shape[-1]
    inv_std, x_hat = _ln_rows(x, cols, eps)
    g = np.asarray(dy, dtype=F32).reshape(-1, cols) * np.asarray(w, dtype=F32).reshape(1, cols)
    s_g = g.sum(axis=1, keepdims=True)
    s_gx = (g * x_hat).sum(axis=1, keepdims=True)
    n = F32(cols)
    dx = (inv_std / n) * ((n * g - s_g) - x_hat * s_gx)
    return dx.reshape(x.shape)


def layer_norm_backward_weight(dy: np.ndarray, x: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """LAYER_NORM_BACKWARD_WEIGHT handler (_realize.py:1053-1063): column sums
    of dy * x_hat, f32 [cols]."""
    cols = x.shape[-1]
    _, x_hat = _ln_rows(x, cols, eps)
    return (np.asarray(dy, dtype=F32).reshape(-1, cols) * x_hat).sum(axis=0)


def layer_norm_backward_bias(dy: np.ndarray) -> np.ndarray:
    """LAYER_NORM_BACKWARD_BIAS handler (_realize.py:1066-1072): column sums of dy."""
    d = np.asarray(dy, dtype=F32)
    return d.reshape(-1, d.shape[-1]).sum(axis=0)


# ---------------------------------------------------------------------------
# Optimizer updates (_realize.py:1637-1721).  Each handler mixes Python floats
# with float32 arrays; NumPy 2 casts a Python float operand to float32 at the
# operation (NEP 50), while float-with-float subexpressions such as
# 1 - beta1, lr * weight_decay and 1 - beta1**step are taken in double first.
# The F32(...) casts below make each of those roundings explicit.
# ---------------------------------------------------------------------------


def sgd_update(param, grad, lr: float, weight_decay: float = 0.0) -> np.ndarray:
    """SGD_UPDATE (_realize.py:1637-1643): param - lr*(grad + wd*param); the
    decay term is skipped when wd == 0."""
    p, g = np.asarray(param, F32), np.asarray(grad, F32)
    u = g + F32(weight_decay) * p if weight_decay != 0.0 else g
    return p - F32(lr) * u


def adamw_update_m(m, grad, beta1: float) -> np.ndarray:
    """ADAMW_UPDATE_M (_realize.py:1646-1650): beta1*m + (1-beta1)*grad."""
    return F32(beta1) * np.asarray(m, F32) + F32(1.0 - beta1) * np.asarray(grad, F32)


def adamw_update_v(v, grad, beta2: float) -> np.ndarray:
    """ADAMW_UPDATE_V (_realize.py:1653-1657): beta2*v + (1-beta2)*grad^2."""
    g = np.asarray(grad, F32)
    return F32(beta2) * np.asarray(v, F32) + F32(1.0 - beta2) * (g * g)


def adamw_update_param(param, m_new, v_new, lr: float, beta1: float, beta2: float, eps: float,
                       step: int, weight_decay: float = 0.0) -> np.ndarray:
    """ADAMW_UPDATE_PARAM (_realize.py:1660-1677): decoupled decay,
    (param - lr*m_hat/(sqrt(v_hat)+eps)) - (lr*wd)*param with
    m_hat = m/(1-beta1^step), v_hat = v/(1-beta2^step)."""
    p = np.asarray(param, F32)
    m_hat = np.asarray(m_new, F32) / F32(1.0 - beta1 ** int(step))
    v_hat = np.asarray(v_new, F32) / F32(1.0 - beta2 ** int(step))
    upd = m_hat / (np.sqrt(v_hat) + F32(eps))
    return (p - F32(lr) * upd) - F32(lr * weight_decay) * p


def _adam_grad(param, grad, weight_decay: float) -> np.ndarray:
    g = np.asarray(grad, F32)
    return g + F32(weight_decay) * np.asarray(param, F32) if weight_decay != 0.0 else g


def adam_update_m(param, grad, m, beta1: float, weight_decay: float = 0.0) -> np.ndarray:
    """ADAM_UPDATE_M (_realize.py:1680-1690): L2 decay folded into the
    gradient, beta1*m + (1-beta1)*(grad + wd*param)."""
    return F32(beta1) * np.asarray(m, F32) + F32(1.0 - beta1) * _adam_grad(param, grad, weight_decay)


def adam_update_v(param, grad, v, beta2: float, weight_decay: float = 0.0) -> np.ndarray:
    """ADAM_UPDATE_V (_realize.py:1693-1703): beta2*v + (1-beta2)*(grad + wd*param)^2."""
    ge = _adam_grad(param, grad, weight_decay)
    return F32(beta2) * np.asarray(v, F32) + F32(1.0 - beta2) * (ge * ge)


def adam_update_param(param, m_new, v_new, lr: float, beta1: float, beta2: float, eps: float,
                      step: int) -> np.ndarray:
    """ADAM_UPDATE_PARAM (_realize.py:1706-1721): param - lr*(m_hat/(sqrt(v_hat)+eps))."""
    m_hat = np.asarray(m_new, F32) / F32(1.0 - beta1 ** int(step))
    v_hat = np.asarray(v_new, F32) / F32(1.0 - beta2 ** int(step))
    return np.asarray(param, F32) - F32(lr) * (m_hat / (np.sqrt(v_hat) + F32(eps)))


# ---------------------------------------------------------------------------
# Convolutions (_realize.py:413-1005): N-d restatements of the per-rank
# handlers.  x [n, c, *in], weight [o, c/groups, *k]; every tap whose input
# index falls outside [0, in) contributes nothing (the handlers pad with zeros
# by `pad` and the transposed handler bounds-checks each output index), and
# the output sizes are taken as given.  Products and sums are float32; the
# reduction order is NumPy's (einsum), not the handlers' loop order.
# ---------------------------------------------------------------------------


def _tap_slices(offset, out_len, stride):
    return slice(offset, offset + (out_len - 1) * stride + 1, stride)


def _padded(x, pad, need):
    """x zero-padded by pad[i] in front of spatial dim i and far enough
    behind that index need[i] - 1 exists."""
    widths = [(0, 0), (0, 0)]
    for i, p in enumerate(pad):
        hi = max(p, need[i] - x.shape[2 + i] - p)
        widths.append((p, hi))
    return np.pad(np.asarray(x, F32), widths)


def _kernel_taps(k):
    return list(np.ndindex(*k))


def _conv_columns(x, k, stride, pad, dil, out):
    """cols[n, c, tap, *out] = x[n, c, out*stride + tap*dil - pad] (0 outside)."""
    need = [(out[i] - 1) * stride[i] + (k[i] - 1) * dil[i] + 1 for i in range(len(k))]
    xp = _padded(x, pad, need)
    taps = []
    for t in _kernel_taps(k):
        sl = tuple(_tap_slices(t[i] * dil[i], out[i], stride[i]) for i in range(len(k)))
        taps.append(xp[(slice(None), slice(None)) + sl])
    return np.stack(taps, axis=2)


def conv_forward(x, w, bias, stride, pad, dil, groups, out):
    """CONV1D / CONV2D / CONV3D (_realize.py:413-450, 532-583, 815-878):
    y[n, g*opg + o, p] = sum_{c, tap} x[n, g*cpg + c, p*s + tap*d - pad] * w[g*opg + o, c, tap] (+ bias)."""
    x = np.asarray(x, F32)
    w = np.asarray(w, F32)
    n, c = x.shape[:2]
    o = w.shape[0]
    k = w.shape[2:]
    cols = _conv_columns(x, k, stride, pad, dil, out)  # [n, c, taps, *out]
    cpg, opg = c // groups, o // groups
    ys = []
    for g in range(groups):
        cg = cols[:, g * cpg:(g + 1) * cpg].reshape(n, cpg * len(_kernel_taps(k)), -1)
        wg = w[g * opg:(g + 1) * opg].reshape(opg, -1)
        ys.append(np.einsum("ok,nkp->nop", wg, cg))
    y = np.concatenate(ys, axis=1).reshape((n, o) + tuple(out)).astype(F32)
    if bias is not None:
        y = y + np.asarray(bias, F32).reshape((1, o) + (1,) * len(k))
    return y


def conv_backward_input(dy, w, stride, pad, dil, groups, in_size):
    """CONV*_BACKWARD_INPUT (_realize.py:452-488, 585-636, 880-941): every
    dy[n, g*opg + o, p] * w[g*opg + o, c, tap] is added into
    dx[n, g*cpg + c, p*s + tap*d - pad]; taps outside [0, in) are dropped."""
    dy = np.asarray(dy, F32)
    w = np.asarray(w, F32)
    n, o = dy.shape[:2]
    out = dy.shape[2:]
    cpg = w.shape[1]
    k = w.shape[2:]
    opg = o // groups
    r = len(k)
    full = [max(in_size[i] + 2 * pad[i], (out[i] - 1) * stride[i] + (k[i] - 1) * dil[i] + 1) for i in range(r)]
    dxp = np.zeros((n, cpg * groups) + tuple(full), F32)
    for ti, t in enumerate(_kernel_taps(k)):
        sl = tuple(_tap_slices(t[i] * dil[i], out[i], stride[i]) for i in range(r))
        for g in range(groups):
            wt = w[g * opg:(g + 1) * opg][(slice(None), slice(None)) + tuple(t)]  # [opg, cpg]
            contrib = np.einsum("oc,no...->nc...", wt, dy[:, g * opg:(g + 1) * opg])
            dxp[(slice(None), slice(g * cpg, (g + 1) * cpg)) + sl] += contrib
    crop = tuple(slice(pad[i], pad[i] + in_size[i]) for i in range(r))
    return dxp[(slice(None), slice(None)) + crop].copy()


def conv_backward_weight(dy, x, k, stride, pad, dil, groups):
    """CONV*_BACKWARD_WEIGHT (_realize.py:490-525, 638-681, 943-1001):
    dw[g*opg + o, c, tap] = sum_{n, p} dy[n, g*opg + o, p] * x[n, g*cpg + c, p*s + tap*d - pad]."""
    dy = np.asarray(dy, F32)
    x = np.asarray(x, F32)
    n, o = dy.shape[:2]
    out = dy.shape[2:]
    c = x.shape[1]
    cols = _conv_columns(x, k, stride, pad, dil, out)
    cpg, opg = c // groups, o // groups
    ntap = len(_kernel_taps(k))
    ws = []
    for g in range(groups):
        cg = cols[:, g * cpg:(g + 1) * cpg].reshape(n, cpg * ntap, -1)
        dg = dy[:, g * opg:(g + 1) * opg].reshape(n, opg, -1)
        ws.append(np.einsum("nop,nkp->ok", dg, cg))
    return np.concatenate(ws, axis=0).reshape((o, cpg) + tuple(k)).astype(F32)


def conv_backward_bias(dy):
    """CONV*_BACKWARD_BIAS (_realize.py:527-529, 683-685, 1003-1005): sum over n and space."""
    dy = np.asarray(dy, F32)
    return dy.sum(axis=(0,) + tuple(range(2, dy.ndim)))


def conv_transpose_forward(x, w, bias, stride, pad, dil, groups, out):
    """CONV_TRANSPOSE2D (_realize.py:712-744): x [n, ci, *in], w [ci, co/groups, *k];
    x[n, ci, p] * w[ci, co', tap] lands on y[n, g*co_pg + co', p*s - pad + tap*d]
    (output indices outside [0, out) dropped), then + bias."""
    y = conv_backward_input(x, w, stride, pad, dil, groups, out)
    if bias is not None:
        y = y + np.asarray(bias, F32).reshape((1, -1) + (1,) * (y.ndim - 2))
    return y


def conv_transpose_backward_input(dy, w, stride, pad, dil, groups, in_size):
    """CONV_TRANSPOSE2D_BACKWARD_INPUT (_realize.py:747-776): the forward
    convolution of dy with the same weight."""
    return conv_forward(dy, w, None, stride, pad, dil, groups, in_size)


def conv_transpose_backward_weight(dy, x, k, stride, pad, dil, groups):
    """CONV_TRANSPOSE2D_BACKWARD_WEIGHT (_realize.py:779-807):
    dw[ci, co', tap] = sum_{n, p} x[n, ci, p] * dy[n, g*co_pg + co', p*s - pad + tap*d]."""
    return conv_backward_weight(x, dy, k, stride, pad, dil, groups)


GELU_C = F32((2.0 / np.pi) ** 0.5)


def gelu_tanh_f32(x: np.ndarray) -> np.ndarray:
    """tanh-GELU exactly as the reference graph evaluates it under autocast
    (_functional.py:115-134): every constant CAST to f32, every op one f32
    ufunc: 0.5*x * (1 + (e^u - e^-u)/(e^u + e^-u)), u = c*(x + 0.044715*x*x*x)."""
    x = np.asarray(x, dtype=F32)
    with np.errstate(all="ignore"):
        half_x = F32(0.5) * x
        cube = F32(0.044715) * x
        cube = cube * x
        cube = cube * x
        inner = x + cube
        u = GELU_C * inner
        ep = np.exp(u)
        en = np.exp(-u)
        th = (ep + (-en)) / (ep + en)
        return half_x * (F32(1.0) + th)


def softmax_lastaxis(x: np.ndarray) -> np.ndarray:
    """Reference softmax graph (_functional.py:152-166): REDUCE max keepdims,
    ADD(x, NEG(max)), EXP, REDUCE sum keepdims, DIV."""
    with np.errstate(all="ignore"):
        m = x.max(axis=-1, keepdims=True)
        e = np.exp(x + (-m))
        return e / e.sum(axis=-1, keepdims=True)


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------


def sdpa_amp(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool) -> np.ndarray:
    """F.scaled_dot_product_attention under autocast (_functional.py:1505-1533):
    scores = f16(q @ k^T) -> f32 * scale -> masked_fill(triu(k=1), -inf) ->
    f32 softmax -> P cast to f16 -> f16(P @ v).  Evaluated per (batch, head)
    slice, which gives identical values (every op is row-local and NumPy's
    batched matmul runs per 2-D slice) at a fraction of the memory."""
    q16, k16, v16 = q.astype(F16), k.astype(F16), v.astype(F16)
    lead = q.shape[:-2]
    sq, sk = q.shape[-2], k.shape[-2]
    out = np.empty(lead + (sq, v.shape[-1]), dtype=F16)
    mask = np.triu(np.ones((sq, sk), dtype=bool), k=1) if causal else None
    s32 = F32(scale)
    for idx in np.ndindex(*lead):
        s = matmul(q16[idx], np.ascontiguousarray(k16[idx].T)).astype(F32) * s32
        if mask is not None:
            s = np.where(mask, F32(-np.inf), s).astype(F32)
        p = softmax_lastaxis(s)
        out[idx] = matmul(p.astype(F16), v16[idx])
    return out


def sdpa_bf16(q_bits, k_bits, v_bits, scale: float, causal: bool) -> np.ndarray:
    """bf16 analogue of sdpa_amp (extension; bit patterns in and out)."""
    q, k, v = (bf16_bits_to_f32(t) for t in (q_bits, k_bits, v_bits))
    lead = q.shape[:-2]
    sq, sk = q.shape[-2], k.shape[-2]
    out = np.empty(lead + (sq, v.shape[-1]), dtype=np.uint16)
    mask = np.triu(np.ones((sq, sk), dtype=bool), k=1) if causal else None
    for idx in np.ndindex(*lead):
        s = round_bf16(q[idx] @ k[idx].T) * F32(scale)
        if mask is not None:
            s = np.where(mask, F32(-np.inf), s).astype(F32)
        p = round_bf16(softmax_lastaxis(s))
        out[idx] = f32_to_bf16_bits(p @ v[idx])
    return out


def attention_online_f32(q, k, v, scale, mask=None):
    """Legacy row-wise online attention (flash_attention.ts:99-129), f32:
    m0 = -1e20, per-key online update, inv_l = l > 0 ? 1/l : 0.  Vectorised
    over rows with float64 accumulation of the same recurrence (pinned by
    the float64 brute-force softmax attention)."""
    s = (q.astype(np.float64) @ np.swapaxes(k.astype(np.float64), -1, -2)) * float(scale)
    if mask is not None:
        s = s + mask.astype(np.float64)
    m = np.maximum(s.max(axis=-1, keepdims=True), -1.0e20)
    p = np.exp(s - m)
    l = p.sum(axis=-1, keepdims=True)
    inv = np.where(l > 0, 1.0 / np.where(l > 0, l, 1.0), 0.0)
    return ((p @ v.astype(np.float64)) * inv).astype(F32)


def attention_forward_f32(q, k, v, scale):
    """Typed ATTENTION_FORWARD in float32, step for step as
    _framework_contracts.py:2906-2929 (execute_attention_forward_arrays):
    scores = q @ k^T (f32 matmul), * f32(scale), row max, exp(scores - max),
    f32 row sum, divide, @ v.  Pinned by attention_f64 (tests)."""
    q, k, v = (np.asarray(t, dtype=F32) for t in (q, k, v))
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        scores = np.matmul(q, np.swapaxes(k, -1, -2))
        scores = np.asarray(scores * np.float32(scale), dtype=F32)
        e = np.exp(scores - scores.max(axis=-1, keepdims=True))
        den = e.sum(axis=-1, keepdims=True, dtype=F32)
        return np.array(np.matmul(e / den, v), dtype=F32)


def attention_f64(q, k, v, scale, causal=False):
    """Brute-force float64 softmax attention (the mathematical definition)."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    s = q @ np.swapaxes(k, -1, -2) * scale
    if causal:
        sq, sk = s.shape[-2], s.shape[-1]
        s = np.where(np.triu(np.ones((sq, sk), bool), 1), -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return p @ v


# ---------------------------------------------------------------------------
# Tolerance rule (semantic-core/src/kernel/attention-forward-model.ts:25-29)
# ---------------------------------------------------------------------------


def within(y, r, tol):
    """abs-or-rel: |y - r| <= tol or |y - r| <= tol * |r|, elementwise."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    d = np.abs(y - r)
    ok = (d <= tol) | (d <= tol * np.abs(r))
    same_nonfinite = (~np.isfinite(y)) & (~np.isfinite(r)) & ((y == r) | (np.isnan(y) & np.isnan(r)))
    return ok | same_nonfinite


def report(y, r, tol):
    ok = within(y, r, tol)
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    fin = np.isfinite(r) & np.isfinite(y)
    d = np.abs(y - r)[fin] if fin.any() else np.zeros(1)
    rn = np.abs(r[fin]).max() if fin.any() else 1.0
    return {
        "pass": bool(ok.all()),
        "n_bad": int((~ok).sum()),
        "max_abs": float(d.max()) if d.size else 0.0,
        "normwise": float(d.max() / rn) if d.size and rn > 0 else 0.0,
    }
