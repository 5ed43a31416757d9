"""GGUF residency on the GPU: tensors read from a GGUF v3 file (written here,
with the reference's byte layout), uploaded once with oco_gguf_upload, and
used in place by the matvec -- results against the oracle on the file bytes."""
import numpy as np
import pytest

import gguf_writer as G
import oracle as O
from _util import Guarded, rel_l2, say

pytestmark = pytest.mark.gpu


def test_gguf_tensors_upload_and_multiply(lib, tmp_path):
    from oco_amd import synth
    specs = [("blk.0.ffn_up.weight", 12, 4096, 300), ("blk.0.ffn_down.weight", 14, 1024, 257),
             ("blk.0.attn_q.weight", 8, 2048, 96), ("blk.0.ffn_gate_exps.weight", 39, 2880, 33)]
    tensors, raw = [], {}
    for name, fmt, k, n in specs:
        data = synth.weights(fmt, n, k, seed=len(name))
        raw[name] = data
        # GGUF shape convention: [input, output] (load.rs:175-186)
        tensors.append((name, [k, n], fmt, data.tobytes()))
    path = tmp_path / "model.gguf"
    path.write_bytes(G.build(metadata=[("general.architecture", G.STRING, "qwen3")], tensors=tensors))
    with lib.Gguf(str(path), ["general.architecture"]) as g:
        assert g.text("general.architecture") == "qwen3"
        d = g.directory()
        for name, fmt, k, n in specs:
            say("gguf", name)
            t = g.select(d[name])
            assert (t.format, t.shape[0], t.shape[1], t.bytes) == (fmt, k, n, raw[name].nbytes)
            w = g.upload(t)
            assert np.array_equal(w.download(np.uint8), raw[name])
            x = synth.activations(k, k)
            y = Guarded(lib, n * 4)
            lib.matvec(fmt, w, lib.DeviceBuffer.from_array(x), y.ptr, lib.Matrix(k, n, 1, 0, 1, 1, 0))
            lib.synchronize()
            want, _ = O.matvec_f64(fmt, raw[name], x, O.Matrix(k, n, 1, 0, 1, 1, 0))
            assert rel_l2(y.read(np.float32), want) <= 1e-5
