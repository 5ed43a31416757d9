#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-weight matrix path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-extra] [--no-cpu]

Prints ONE JSON line.  The headline (``value``) is the workload BASELINE's
metric is quoted on at one GPU: the MXFP4 decode matvec at gpt-oss-20b's
expert shape (weight [5760 x 2880], one f32 activation vector, fp32
accumulation), in GB/s of streamed weight bytes.  A step is one launch of
the fused dequantize+matvec over one weight copy; inputs are resident in HBM
before timing starts.  The weight is replicated into enough distinct copies
(> 512 MiB) that successive steps rotate through them, so the 256 MB
Infinity Cache cannot serve repeats (the reference rotates weight copies for
the same reason, dense_bench.rs:220-250).  The K timed steps are one
captured HIP graph, replayed after W warmup steps, bracketed by device
synchronisation; HIP events on the launch stream time the region.

``extra`` carries the other BASELINE configs measured the same way.
``cpu_baseline`` times the scalar C oracle (dequantize-then-fp32-dot, the
"port" of the reference's semantics) on the host on the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, AMD published
MALL_BYTES = 256 * 2 ** 20     # Infinity Cache
ROTATE_BYTES = 512 * 2 ** 20   # distinct weight bytes a timed step sequence cycles through


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Workload:
    name = ""
    unit = "GB/s"
    bound = "hbm"

    def setup(self, oco, stream):
        raise NotImplementedError

    def launch(self, i: int):
        raise NotImplementedError

    def work_per_step(self) -> float:  # algorithmic bytes (hbm) or flops (mfma)
        raise NotImplementedError


class Matvec(Workload):
    """Fused dequantize + matvec over rotated weight copies."""

    def __init__(self, name, fmt, n, k, seed=1, label=None):
        self.name, self.fmt, self.n, self.k, self.seed = name, fmt, n, k, seed
        self.label = label or name

    def setup(self, oco, stream):
        from oco_amd import synth
        self.oco, self.stream = oco, stream
        data = synth.weights(self.fmt, self.n, self.k, self.seed)
        self.bytes = data.nbytes
        self.copies = max(1, math.ceil(ROTATE_BYTES / self.bytes))
        self.w = oco.DeviceBuffer(self.bytes * self.copies)
        self.w.upload(data)
        for c in range(1, self.copies):
            oco.load_library().oco_buffer_copy(self.w.ptr + c * self.bytes, self.w.ptr, self.bytes,
                                               stream.handle)
        stream.sync()
        self.x = oco.DeviceBuffer.from_array(synth.activations(self.seed + 1, self.k))
        self.y = oco.DeviceBuffer(self.n * 4)
        self.p = oco.Matrix(self.k, self.n, 1, 0, 1, 1, 0)

    def launch(self, i):
        self.oco.matvec(self.fmt, self.w.ptr + (i % self.copies) * self.bytes, self.x, self.y,
                        self.p, stream=self.stream)

    def work_per_step(self):
        return float(self.bytes)


class ReadFloor(Workload):
    """The plain HBM read stream the decode matvec is bounded by: the XOR of
    every word of the headline's 8,812,800 weight bytes (oco_buffer_xor32,
    four 16-byte nontemporal loads in flight per thread), over the same
    rotated copies.  Work = bytes read."""
    name = "read_floor_8812800"

    def setup(self, oco, stream):
        from oco_amd import synth
        self.oco, self.stream = oco, stream
        data = synth.weights(39, 5760, 2880, 1)
        self.bytes = data.nbytes
        self.copies = max(1, math.ceil(ROTATE_BYTES / self.bytes))
        self.stride = (self.bytes + 255) // 256 * 256
        self.w = oco.DeviceBuffer(self.stride * self.copies)
        for c in range(self.copies):
            self.w.upload(data, c * self.stride)
        self.out = oco.DeviceBuffer(4096)

    def launch(self, i):
        self.w.xor32(self.out, stream=self.stream, offset=(i % self.copies) * self.stride, nbytes=self.bytes)

    def work_per_step(self):
        return float(self.bytes)


class MatvecStack(Workload):
    """Qwen3-8B-shaped decode stack: ffn_up/gate Q4_K (one grouped launch, the
    reference's concurrent pair), ffn_down Q6_K, lm_head Q6_K."""
    name = "qwen3_8b_q4km_decode_stack"

    def setup(self, oco, stream):
        from oco_amd import synth
        self.oco, self.stream = oco, stream
        self.mats = []
        for fmt, n, k, seed in [(12, 12288, 4096, 31), (12, 12288, 4096, 32), (14, 4096, 12288, 33),
                                (14, 151936, 4096, 34)]:
            data = synth.weights(fmt, n, k, seed)
            self.mats.append((fmt, n, k, oco.DeviceBuffer.from_array(data), data.nbytes))
        self.bytes = sum(m[4] for m in self.mats)
        self.x = oco.DeviceBuffer.from_array(synth.activations(35, 12288))
        self.h = oco.DeviceBuffer(151936 * 4)
        self.h2 = oco.DeviceBuffer(12288 * 4)

    def launch(self, i):
        o = self.oco
        (fu, nu, ku, wu, _), (_, _, _, wg, _) = self.mats[:2]
        o.matvec_group(fu, [wu, wg], self.x, [self.h, self.h2], o.Matrix(ku, nu, 1, 0, 1, 1, 0), o.DType.F32,
                       stream=self.stream)
        for fmt, n, k, w, nb in self.mats[2:]:
            o.matvec(fmt, w, self.x, self.h, o.Matrix(k, n, 1, 0, 1, 1, 0), stream=self.stream)

    def work_per_step(self):
        return float(self.bytes)


class LmHeadArgmax(Workload):
    """The decode tail: Qwen3-8B lm_head [151936 x 4096] Q6_K with f32 logits,
    then greedy argmax over them (Compute::argmax, compute.rs:132-140).
    Work = lm_head weight bytes (the logits add 0.6 MB)."""
    name = "lm_head_argmax_qwen3_8b"

    def setup(self, oco, stream):
        from oco_amd import synth
        self.oco, self.stream = oco, stream
        self.n, self.k = 151936, 4096
        data = synth.weights(14, self.n, self.k, 34)
        self.bytes = data.nbytes
        self.w = oco.DeviceBuffer.from_array(data)
        self.x = oco.DeviceBuffer.from_array(synth.activations(36, self.k))
        self.y = oco.DeviceBuffer(self.n * 4)
        self.tok = oco.DeviceBuffer(4)
        self.ws_bytes = oco.argmax_workspace(self.n)
        self.ws = oco.DeviceBuffer(max(self.ws_bytes, 4))
        self.p = oco.Matrix(self.k, self.n, 1, 0, 1, 1, 0)

    def launch(self, i):
        self.oco.matvec(14, self.w, self.x, self.y, self.p, stream=self.stream)
        self.oco.argmax(self.y, self.n, self.tok, stream=self.stream, workspace=self.ws,
                        workspace_bytes=self.ws_bytes)

    def work_per_step(self):
        return float(self.bytes)


class Argmax(Workload):
    """argmax over Qwen3-8B's 151936 f32 logits alone (latency-bound; GB/s of logits)."""
    name = "argmax_f32_151936"

    def setup(self, oco, stream):
        import numpy as np
        self.oco, self.stream = oco, stream
        self.n = 151936
        self.y = oco.DeviceBuffer.from_array(np.random.default_rng(1).normal(size=self.n).astype(np.float32))
        self.tok = oco.DeviceBuffer(4)
        self.ws_bytes = oco.argmax_workspace(self.n)
        self.ws = oco.DeviceBuffer(max(self.ws_bytes, 4))

    def launch(self, i):
        self.oco.argmax(self.y, self.n, self.tok, stream=self.stream, workspace=self.ws,
                        workspace_bytes=self.ws_bytes)

    def work_per_step(self):
        return float(self.n * 4)


class NormUpGate(Workload):
    """Qwen3-8B FFN entry: RMS norm of the bf16 residual row, then ffn_up and
    ffn_gate [12288 x 4096] Q4_K.  mode "group": the norm and both matrices
    in one grid (oco_matvec_group, the reference's concurrent up/gate pair);
    "fused": the norm inside each matvec's activation staging
    (oco_matvec_norm), two launches; "unfused": oco_norm then two matvecs.
    The pair is replicated into enough copies (> 512 MiB) that successive
    steps rotate through them past the Infinity Cache.  Work = the two
    weight matrices' bytes."""

    def __init__(self, mode):
        self.mode = mode
        self.name = "norm_up_gate_qwen3_8b_" + mode

    def setup(self, oco, stream):
        import numpy as np
        from oco_amd import synth
        self.oco, self.stream = oco, stream
        self.n, self.k = 12288, 4096
        mats = [synth.weights(12, self.n, self.k, s) for s in (31, 32)]
        self.mbytes = mats[0].nbytes
        self.bytes = 2 * self.mbytes
        self.copies = max(1, math.ceil(ROTATE_BYTES / self.bytes))
        self.w = oco.DeviceBuffer(self.bytes * self.copies)
        self.w.upload(mats[0], 0)
        self.w.upload(mats[1], self.mbytes)
        for c in range(1, self.copies):
            oco.load_library().oco_buffer_copy(self.w.ptr + c * self.bytes, self.w.ptr, self.bytes, stream.handle)
        stream.sync()
        self.x = oco.DeviceBuffer.from_array(synth.bf16_bits(synth.activations(37, self.k)))
        self.nw = oco.DeviceBuffer.from_array((1 + 0.1 * np.random.default_rng(2).normal(size=self.k)).astype(np.float32))
        self.normed = oco.DeviceBuffer(self.k * 2)
        self.y = [oco.DeviceBuffer(self.n * 4) for _ in range(2)]
        self.p = oco.Matrix(self.k, self.n, 1, 0, 1, 1, 0)

    def launch(self, i):
        o = self.oco
        base = self.w.ptr + (i % self.copies) * self.bytes
        mats = [base, base + self.mbytes]
        if self.mode == "group":
            o.matvec_group(12, mats, self.x, self.y, self.p, o.DType.BF16, o.DType.F32, self.nw, 1e-6, True,
                           stream=self.stream)
        elif self.mode == "fused":
            for w, y in zip(mats, self.y):
                o.matvec_norm(12, w, self.x, self.nw, 1e-6, y, self.p, True, stream=self.stream)
        else:
            o.norm(self.x, self.nw, self.normed, 1, self.k, 1e-6, True, stream=self.stream)
            for w, y in zip(mats, self.y):
                o.matvec(12, w, self.normed, y, self.p, o.DType.BF16, stream=self.stream)

    def work_per_step(self):
        return float(self.bytes)


class MoeDecode(Workload):
    """gpt-oss-20b expert layer from the router on (Bindings::experts,
    feed_forward.rs:107-275): router logits over 32 experts (f32 router rows
    scaled so the logits are ~N(0,1)), top-4 with softmax over the chosen,
    gate/up [2880 x 2880] and down [2880 x 2880] MXFP4, clipped SwiGLU,
    weighted combine with residual; `tokens` per step.  Two copies of the
    bank (2 x 423 MB) and 16 activation batches (so 16 routings) rotate so
    successive steps miss the Infinity Cache.  Work = distinct experts hit x
    13,219,200 bytes, counted from the device's own selections."""

    def __init__(self, tokens):
        self.tokens = tokens
        self.name = f"moe_decode_gpt_oss_b{tokens}"

    def setup(self, oco, stream):
        import numpy as np
        from oco_amd import synth
        self.oco, self.stream = oco, stream
        E, h, f, k = 32, 2880, 2880, 4
        self.k = k
        banks = _BANKS.get("gpt_oss")
        if banks is None:
            banks = _BANKS["gpt_oss"] = self._banks(oco, E, h, f, k)
        self.banks = banks
        rng = np.random.default_rng(1234)
        self.router_w = oco.DeviceBuffer.from_array((rng.normal(size=(E, h)) / np.sqrt(h)).astype(np.float32))
        self.router_b = oco.DeviceBuffer.from_array((rng.normal(size=E) * 0.1).astype(np.float32))
        self.x = [oco.DeviceBuffer.from_array(synth.activations(200 + i, self.tokens * h)) for i in range(16)]
        self.out = oco.DeviceBuffer.from_array(np.zeros(self.tokens * h, np.uint16))
        self.ws = oco.DeviceBuffer(banks[0].workspace_bytes(self.tokens))
        self.ids = oco.DeviceBuffer(self.tokens * k * 4)
        self.probs = oco.DeviceBuffer(self.tokens * k * 4)
        self.expert_bytes = 3 * f * (h // 32) * 17
        distinct = []
        for i in range(16):  # the experts each activation batch routes to, as the device selects them
            self.launch(i)
            stream.sync()
            distinct.append(len(set(self.ids.download(np.uint32).tolist())))
        self.distinct = float(np.mean(distinct))

    @staticmethod
    def _banks(oco, E, h, f, k):
        from oco_amd import synth
        banks = []
        for c in range(2):
            g = synth.weights(39, E * f, h, 100 + 3 * c)
            u = synth.weights(39, E * f, h, 101 + 3 * c)
            d = synth.weights(39, E * h, f, 102 + 3 * c)
            rng = np.random.default_rng(c)
            bias = [oco.DeviceBuffer.from_array((rng.normal(size=E * n) * 0.1).astype(np.float32))
                    for n in (f, f, h)]
            bufs = [oco.DeviceBuffer.from_array(a) for a in (g, u, d)]
            banks.append(oco.ExpertBank(39, h, f, E, k, *bufs, *bias))
            del g, u, d
        return banks

    def launch(self, i):
        self.banks[i % 2].forward(self.router_w, self.router_b, self.x[i % 16], self.oco.DType.F32, self.tokens,
                                  self.out, self.ids, self.probs, workspace=self.ws, stream=self.stream)

    def work_per_step(self):
        return self.distinct * self.expert_bytes


class MoePrefill(MoeDecode):
    """Qwen3-30B-A3B expert layer at prefill: 128 experts, gate/up [768 x 2048]
    and down [2048 x 768] Q4_K, top-8 of softmax(N(0,1) logits) over 512
    tokens (4096 routes: every expert is hit), SwiGLU, weighted combine.  Two
    bank copies (2 x 340 MB) rotate past the Infinity Cache.  Work = bytes of
    the experts hit (HBM-bound: 38.65 GFLOP over 339,738,624 bytes)."""

    def __init__(self, tokens=512):
        self.tokens = tokens
        self.name = "moe_prefill_qwen3_30b_a3b"

    def setup(self, oco, stream):
        import numpy as np
        from oco_amd import synth
        self.oco, self.stream = oco, stream
        E, h, f, k = 128, 2048, 768, 8
        self.k = k
        banks = _BANKS.get("qwen3_30b")
        if banks is None:
            banks = _BANKS["qwen3_30b"] = []
            for c in range(2):
                g = synth.weights(12, E * f, h, 300 + 3 * c)
                u = synth.weights(12, E * f, h, 301 + 3 * c)
                d = synth.weights(12, E * h, f, 302 + 3 * c)
                bufs = [oco.DeviceBuffer.from_array(a) for a in (g, u, d)]
                banks.append(oco.ExpertBank(12, h, f, E, k, *bufs, activation=oco.Activation.SWIGLU,
                                            up_bias_one=False))
                del g, u, d
        self.banks = banks
        self.tables = []
        distinct = []
        rng = np.random.default_rng(4321)
        for t in range(8):
            logits = rng.normal(size=(self.tokens, E)).astype(np.float32)
            ids, probs = _select(logits, k)
            distinct.append(len(set(ids.ravel().tolist())))
            self.tables.append((oco.DeviceBuffer.from_array(ids), oco.DeviceBuffer.from_array(probs)))
        self.distinct = float(np.mean(distinct))
        self.x = [oco.DeviceBuffer.from_array(synth.bf16_bits(synth.activations(400 + i, self.tokens * h)))
                  for i in range(2)]
        self.out = oco.DeviceBuffer.from_array(np.zeros(self.tokens * h, np.uint16))
        self.ws = oco.DeviceBuffer(banks[0].workspace_bytes(self.tokens))
        self.expert_bytes = 3 * f * (h // 256) * 144

    def launch(self, i):
        ids, probs = self.tables[i % 8]
        self.banks[i % 2].apply(self.x[i % 2], self.oco.DType.BF16, ids, probs, self.tokens, self.out,
                                workspace=self.ws, stream=self.stream)


_BANKS = {}


def _select(logits, k):
    """Top-k with softmax over the selected (host-side routing tables for the bench)."""
    import numpy as np
    order = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    chosen = np.take_along_axis(logits, order, axis=1)
    p = np.exp(chosen - chosen[:, :1])
    return order.astype(np.uint32), (p / p.sum(axis=1, keepdims=True)).astype(np.float32)


class Prefill(Workload):
    """Dense prefill Y = X W^T on MFMA: weight [n x k] GGUF, `m` bf16 tokens,
    bf16 output rows (the reference's matrix kernels store bf16 unless asked
    for f32: shaders/matrix/weights.metal:24-33)."""
    bound = "mfma"
    unit = "TFLOP/s"

    def __init__(self, name, fmt, n, k, m):
        self.name, self.fmt, self.n, self.k, self.m = name, fmt, n, k, m

    def setup(self, oco, stream):
        from oco_amd import synth
        self.oco, self.stream = oco, stream
        w = synth.weights(self.fmt, self.n, self.k, 7)
        self.bytes = w.nbytes
        self.copies = max(1, math.ceil(ROTATE_BYTES / self.bytes))
        self.w = oco.DeviceBuffer(self.bytes * self.copies)
        for c in range(self.copies):
            self.w.upload(w, c * self.bytes)
        self.x = oco.DeviceBuffer.from_array(synth.bf16_bits(synth.activations(8, self.m * self.k)))
        self.y = oco.DeviceBuffer(self.m * self.n * 2)
        self.p = oco.Matrix(self.k, self.n, self.m, 0, 1, 1, 0)
        self.ws_bytes = oco.matmul_workspace(self.fmt, self.p)
        self.ws = oco.DeviceBuffer(max(self.ws_bytes, 256))

    def launch(self, i):
        self.oco.matmul(self.fmt, self.w.ptr + (i % self.copies) * self.bytes, self.x, self.y, self.p,
                        y_dtype=self.oco.DType.BF16, stream=self.stream, workspace=self.ws, workspace_bytes=self.ws_bytes)

    def work_per_step(self):
        return 2.0 * self.m * self.n * self.k


class NormPrefill(Prefill):
    """The norm -> MXFP4 prefill pair of a layer (prepare_norm_scales +
    apply_norm, feed_forward.rs:99-101): the RMS norm of 512 bf16 residual
    rows, then the 5760 x 2880 MXFP4 product of the normalised rows.
    "fused": oco_norm_mx_split + oco_matmul_mx_split (two launches);
    "unfused": oco_norm + oco_matmul_ws (norm, split, product: three)."""

    def __init__(self, mode):
        super().__init__(f"norm_prefill_mxfp4_5760x2880_m512_{mode}", 39, 5760, 2880, 512)
        self.mode = mode

    def setup(self, oco, stream):
        super().setup(oco, stream)
        import numpy as np
        self.nw = oco.DeviceBuffer.from_array(np.random.default_rng(5).normal(1.0, 0.1, self.k).astype(np.float32))
        self.xn = oco.DeviceBuffer(self.m * self.k * 2)

    def launch(self, i):
        o = self.oco
        w = self.w.ptr + (i % self.copies) * self.bytes
        if self.mode == "fused":
            o.norm_mx_split(self.x, self.nw, None, self.m, self.k, 1e-5, True, self.ws, self.ws_bytes, stream=self.stream)
            o.matmul_mx_split(w, self.ws, self.ws_bytes, self.y, self.p, y_dtype=o.DType.BF16, stream=self.stream)
        else:
            o.norm(self.x, self.nw, self.xn, self.m, self.k, 1e-5, True, stream=self.stream)
            o.matmul(self.fmt, w, self.xn, self.y, self.p, y_dtype=o.DType.BF16, stream=self.stream,
                     workspace=self.ws, workspace_bytes=self.ws_bytes)


WORKLOADS = {
    "mxfp4_decode_matvec_5760x2880": lambda: Matvec("mxfp4_decode_matvec_5760x2880", 39, 5760, 2880),
    "q8_0_matvec_4096x4096": lambda: Matvec("q8_0_matvec_4096x4096", 8, 4096, 4096),
    "q4_k_matvec_12288x4096": lambda: Matvec("q4_k_matvec_12288x4096", 12, 12288, 4096),
    "q6_k_matvec_4096x12288": lambda: Matvec("q6_k_matvec_4096x12288", 14, 4096, 12288),
    "q6_k_lm_head_151936x4096": lambda: Matvec("q6_k_lm_head_151936x4096", 14, 151936, 4096),
    "q4_0_matvec_4096x4096": lambda: Matvec("q4_0_matvec_4096x4096", 2, 4096, 4096),
    "q4_1_matvec_4096x4096": lambda: Matvec("q4_1_matvec_4096x4096", 3, 4096, 4096),
    "q5_k_matvec_12288x4096": lambda: Matvec("q5_k_matvec_12288x4096", 13, 12288, 4096),
    "qwen3_8b_q4km_decode_stack": MatvecStack,
    "read_floor_8812800": ReadFloor,
    "moe_decode_gpt_oss_b1": lambda: MoeDecode(1),
    "moe_decode_gpt_oss_b4": lambda: MoeDecode(4),
    "moe_decode_gpt_oss_b16": lambda: MoeDecode(16),
    "prefill_mxfp4_5760x2880_m512": lambda: Prefill("prefill_mxfp4_5760x2880_m512", 39, 5760, 2880, 512),
    "norm_prefill_mxfp4_5760x2880_m512_fused": lambda: NormPrefill("fused"),
    "norm_prefill_mxfp4_5760x2880_m512_unfused": lambda: NormPrefill("unfused"),
    "prefill_q4_k_12288x4096_m512": lambda: Prefill("prefill_q4_k_12288x4096_m512", 12, 12288, 4096, 512),
    "prefill_q6_k_4096x12288_m512": lambda: Prefill("prefill_q6_k_4096x12288_m512", 14, 4096, 12288, 512),
    "prefill_q8_0_4096x4096_m512": lambda: Prefill("prefill_q8_0_4096x4096_m512", 8, 4096, 4096, 512),
    "moe_prefill_qwen3_30b_a3b": MoePrefill,
    "lm_head_argmax_qwen3_8b": LmHeadArgmax,
    "argmax_f32_151936": Argmax,
    "norm_up_gate_qwen3_8b_group": lambda: NormUpGate("group"),
    "norm_up_gate_qwen3_8b_fused": lambda: NormUpGate("fused"),
    "norm_up_gate_qwen3_8b_unfused": lambda: NormUpGate("unfused"),
}
PEAK_TFLOPS = {"bf16": 2500.0, "fp4": 10100.0}
HEADLINE = "mxfp4_decode_matvec_5760x2880"


def time_workload(oco, wl: Workload, steps: int, warmup: int):
    stream = oco.Stream()
    wl.setup(oco, stream)
    if warmup:
        warm = oco.Graph(stream, lambda: [wl.launch(i) for i in range(warmup)])
        warm.launch()
    graph = oco.Graph(stream, lambda: [wl.launch(warmup + i) for i in range(steps)])
    stream.sync()
    oco.synchronize()
    start, stop = oco.Event(), oco.Event()
    start.record(stream)
    graph.launch()
    stop.record(stream)
    ms = start.elapsed_ms(stop)
    stream.sync()
    oco.synchronize()
    per_step_s = ms / 1e3 / steps
    work = wl.work_per_step()
    achieved = work / per_step_s / (1e12 if wl.unit == "TFLOP/s" else 1e9)
    return {"ms_per_step": ms / steps, "achieved": achieved, "work": work}


def host_cores() -> int:
    """Every core this process may run on: the affinity mask, capped by the
    cgroup's CPU quota when one is set (a quota below the mask means the
    extra threads would only time-share)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return max(1, n)


def cpu_baseline(budget_s: float = 10.0):
    """Scalar C oracle (dequantize-then-fp32-dot) on host cores, same workload."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    from oco_amd import synth
    n, k = 5760, 2880
    w = synth.weights(39, n, k, 1)
    x = synth.activations(2, k)
    threads = host_cores()
    p = O.Matrix(k, n, 1, 0, 1, 1, 0)

    def best_of(nthreads, budget):
        t0 = time.perf_counter()
        O.matvec_f32(39, w, x, p, threads=nthreads)
        best = time.perf_counter() - t0
        end, done = time.perf_counter() + budget, 1
        while time.perf_counter() < end:
            t0 = time.perf_counter()
            O.matvec_f32(39, w, x, p, threads=nthreads)
            best = min(best, time.perf_counter() - t0)
            done += 1
        return best, done

    best, done = best_of(threads, budget_s)
    best1, done1 = best_of(1, budget_s / 4)
    return {"value": round(w.nbytes / best / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "single_thread": round(w.nbytes / best1 / 1e9, 3),
            "sample": f"full MXFP4 5760x2880 matvec (8,812,800 weight bytes), best of {done} runs "
                      f"over ~{budget_s:.0f} s, OpenMP {threads} threads (every core of the job's affinity "
                      f"and CPU quota), C oracle -O3; "
                      f"single_thread: best of {done1} runs on one thread"}


def load_traffic(name: str):
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default=HEADLINE, choices=sorted(WORKLOADS))
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 10 device copies of 256 MiB (counter calibration for traffic)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build runs its kernels on a single MI355X "
              "(multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import oco_amd as oco
    cus = oco.open_device(0)
    log(f"device 0: {cus} CUs")
    if args.calibrate_copy:
        n = 256 * 2 ** 20
        src, dst = oco.DeviceBuffer(n), oco.DeviceBuffer(n)
        src.fill32(0x01020304)
        for _ in range(10):
            oco.load_library().oco_buffer_copy(dst.ptr, src.ptr, n, None)
        oco.synchronize()
        print(json.dumps({"calibrate_copy_bytes": n, "copies": 10}))
        return

    wl = WORKLOADS[args.workload]()
    log(f"timing {wl.name}: {args.steps} steps after {args.warmup} warmup")
    r = time_workload(oco, wl, args.steps, args.warmup)
    value = r["achieved"]
    traffic = load_traffic(wl.name)
    is_flops = wl.unit == "TFLOP/s"
    # MXFP4 prefill is priced against the block-scaled FP4 MFMA peak, other
    # prefill against bf16, decode against HBM
    peak = (PEAK_TFLOPS["fp4" if getattr(wl, "fmt", None) == 39 else "bf16"] if is_flops else HBM_PEAK_GBS)
    out = {
        "metric": ("prefill TFLOP/s (% MFMA)" if is_flops
                   else "weight GB/s (% of HBM peak) for decode matvec"),
        "value": round(value, 2),
        "unit": wl.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("fp6 x fp4 block-scaled MFMA (bf16 activations as two E2M3 terms), f32 accumulation"
                  if is_flops and getattr(wl, "fmt", None) == 39 else "f16 MFMA, f32 accumulation" if is_flops else "f32"),
        "data": "synthetic (seeded GGUF-layout weights, N(0,1) activations)",
        "config": {"workload": wl.name, "format": getattr(wl, "fmt", None), "n": getattr(wl, "n", None),
                   "k": getattr(wl, "k", None), "batch": getattr(wl, "m", getattr(wl, "tokens", 1)),
                   ("flops" if is_flops else "weight_bytes"): int(r["work"]),
                   "rotated_copies": getattr(wl, "copies", 1)},
        "roofline": {"bound": wl.bound, "achieved": round(value, 2),
                     "peak": peak, "unit": wl.unit, "frac": round(value / peak, 4),
                     "traffic": traffic},
    }
    if not args.no_extra:
        extra = []
        for name in ["q8_0_matvec_4096x4096", "q4_k_matvec_12288x4096", "q6_k_matvec_4096x12288",
                     "q6_k_lm_head_151936x4096", "qwen3_8b_q4km_decode_stack", "moe_decode_gpt_oss_b1",
                     "moe_decode_gpt_oss_b4", "moe_decode_gpt_oss_b16", "prefill_mxfp4_5760x2880_m512",
                     "norm_prefill_mxfp4_5760x2880_m512_fused", "norm_prefill_mxfp4_5760x2880_m512_unfused",
                     "prefill_q4_k_12288x4096_m512", "prefill_q6_k_4096x12288_m512", "prefill_q8_0_4096x4096_m512",
                     "moe_prefill_qwen3_30b_a3b", "lm_head_argmax_qwen3_8b", "argmax_f32_151936",
                     "norm_up_gate_qwen3_8b_group", "norm_up_gate_qwen3_8b_fused",
                     "norm_up_gate_qwen3_8b_unfused", "read_floor_8812800"]:
            if name == wl.name:
                continue
            w2 = WORKLOADS[name]()
            steps = max(20, min(args.steps, 200))
            log(f"timing {name}: {steps} steps")
            r2 = time_workload(oco, w2, steps, min(args.warmup, 10))
            entry = {"workload": name, "value": round(r2["achieved"], 2), "unit": w2.unit,
                     "ms_per_step": round(r2["ms_per_step"], 6)}
            if w2.unit == "GB/s":
                entry.update(frac=round(r2["achieved"] / HBM_PEAK_GBS, 4), work_bytes=int(r2["work"]))
            else:
                entry.update(frac_bf16_mfma=round(r2["achieved"] / PEAK_TFLOPS["bf16"], 4),
                             frac_fp4_mfma=round(r2["achieved"] / PEAK_TFLOPS["fp4"], 4),
                             work_flops=int(r2["work"]))
            extra.append(entry)
            del w2
        out["extra"] = extra
    if not args.no_cpu:
        log("cpu baseline (C oracle)")
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
