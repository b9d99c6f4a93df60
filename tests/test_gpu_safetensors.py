"""GPT-2 block weights loaded from safetensors straight into device memory
(load_safetensors_resident), then realized by the walker (GPU).

The block is the C5 GPT-2 block at reduced size with Hugging Face-named
weights written by the safetensors package; the walker's output is compared
with the graph oracle (f16 autocast tolerance 2e-2), and the walk performs
no weight upload of its own (the resident loader put every weight in the
GpuBufferTable; only the activation input is uploaded)."""
from __future__ import annotations

import numpy as np
import pytest
import safetensors.numpy as stnp

from browsergrad_amd.jit import configs
from browsergrad_amd.jit.buffers import GpuBufferTable
from browsergrad_amd.jit.realize import realize_hip
from browsergrad_amd.jit.safetensors import gpt2_block_params, load_safetensors_resident
from browsergrad_amd.jit.tensor import Session, autocast
from oracle import graph as G
from oracle import ops as O

pytestmark = pytest.mark.gpu


def test_gpt2_block_from_resident_safetensors(bridge, tmp_path):
    rng = np.random.default_rng(11)
    heads, emb, bsz, seq = 4, 256, 2, 64
    f = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float32)  # noqa: E731
    hf = {
        "h.0.ln_1.weight": (1 + f(emb)), "h.0.ln_1.bias": f(emb),
        "h.0.attn.c_attn.weight": f(emb, 3 * emb), "h.0.attn.c_attn.bias": f(3 * emb),
        "h.0.attn.c_proj.weight": f(emb, emb), "h.0.attn.c_proj.bias": f(emb),
        "h.0.ln_2.weight": (1 + f(emb)), "h.0.ln_2.bias": f(emb),
        "h.0.mlp.c_fc.weight": f(emb, 4 * emb), "h.0.mlp.c_fc.bias": f(4 * emb),
        "h.0.mlp.c_proj.weight": f(4 * emb, emb), "h.0.mlp.c_proj.bias": f(emb),
    }
    path = tmp_path / "gpt2_block.safetensors"
    stnp.save_file(hf, str(path))
    s = Session()
    gbt = GpuBufferTable(bridge)
    c0 = dict(bridge.counters)
    tensors = load_safetensors_resident(str(path), gbt, session=s)
    assert bridge.counters["upload"] - c0["upload"] == len(hf)
    for name, arr in hf.items():
        h = gbt.get(tensors[name].uop.inputs[0].arg)
        assert np.array_equal(bridge.to_numpy(h), arr), name
    x = rng.standard_normal((bsz, seq, emb)).astype(np.float32)
    with autocast("float16"):
        y = configs.gpt2_block(s.from_numpy(x, "x"), gpt2_block_params(tensors, 0), heads)
    ref = G.evaluate(y.uop, s.buffers)
    c1 = dict(bridge.counters)
    out = realize_hip(y.uop, s.buffers, gbt)
    assert bridge.counters["upload"] - c1["upload"] == 1  # x only
    rep = O.report(out.astype(np.float32), ref.astype(np.float32), 2e-2)
    assert rep["pass"], rep
    gbt.release_all()
