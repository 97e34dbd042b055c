"""Benchmark: achieved HBM bandwidth of emel.rs's elementwise, broadcast and
row-reduction ops on one MI355X (BASELINE.json metric).

One step = one launch of every op of the five BASELINE configs, each on its
own buffers (no op reads another op's output), so each launch streams cold
data from HBM: between two launches of the same op the other ops move
~1 GB, far more than the 256 MB Infinity Cache.  Inputs are synthetic
(seeded PCG64) and already resident in HBM when the timed region starts.

Times come from HIP events recorded on the stream the kernels run on.  The
steps are captured once into a HIP graph and replayed (removing Python
launch overhead, which is larger than the smaller kernels); the replays
are checked bit-for-bit against eager launches, and the eager step time is
reported beside.  The value is total algorithmic bytes per step / step
time.  Each op's own figure is the average over a graph of back-to-back
launches of that op that cycle through at least 1 GiB of distinct buffer
sets, so those launches are cold too.  The roofline object describes the
dominant kernel (the scaled + masked soft_max of config 4, over half of the
step's bytes).  The CPU baseline times the C oracle (a single-threaded
restatement of the reference's CPU path) on the same config tensors: one
warm-up run, then the median of 5.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--ops a,b] [--no-cpu] [--no-copy] [--pcie] [--no-gather]
                    [--no-sampler] [--launches N]

--launches N only launches each op (and the calibration copy) N times, for
rocprofv3 counter runs; config.launch_floor_us is the per-launch time of
back-to-back launches that move almost no bytes.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "emel.rs_amd", ROOT / "oracle"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "achieved HBM GB/s and % of 8 TB/s peak per op (binary, rms_norm, softmax)"
PEAK_GBS = 8000.0
MB = 1e6


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def normal(seed, n, sigma=1.0):
    return (rng(seed).standard_normal(n, dtype=np.float64) * sigma).astype(np.float32)


def uniform(seed, n, lo, hi):
    return rng(seed).uniform(lo, hi, n).astype(np.float32)


def causal_mask(nkv, nq):
    k = np.arange(nkv)[None, :]
    q = np.arange(nq)[:, None]
    return np.where(k <= q + (nkv - nq), np.float16(0.0), np.float16(-np.inf)).astype(np.float16).reshape(-1)


def config_inputs():
    """Host arrays of the BASELINE configs (seeded)."""
    d = {}
    # config 1: [4096,512] + [4096], U(-1,1)
    d["c1_src0"] = uniform(1, 4096 * 512, -1, 1)
    d["c1_src1"] = uniform(2, 4096, -1, 1)
    # config 2: gate, up [11008,512] N(0,1)
    d["c2_gate"] = normal(3, 11008 * 512)
    d["c2_up"] = normal(4, 11008 * 512)
    # config 3: x [4096,2048] N(0,1), 1% of rows x100; w [4096] U(0.5,1.5)
    x = normal(5, 4096 * 2048).reshape(2048, 4096)
    x[rng(6).choice(2048, 20, replace=False)] *= np.float32(100.0)
    d["c3_x"] = x.reshape(-1)
    d["c3_w"] = uniform(7, 4096, 0.5, 1.5)
    # config 4: scores [4096,512,32] N(0,4), causal f16 mask [4096,512]
    d["c4_x"] = normal(8, 4096 * 512 * 32, 2.0)
    d["c4_mask"] = causal_mask(4096, 512).view(np.uint16)
    # config 5: logits [151936,64] N(0,1) with a planted max per row (+ ties)
    lg = normal(9, 151936 * 64).reshape(64, 151936)
    g = rng(10)
    where = g.integers(0, 151936, 64)
    for r in range(64):
        lg[r, where[r]] = np.float32(8.0)
        if r % 2 == 0 and where[r] + 1 < 151936:
            lg[r, g.integers(where[r] + 1, 151936)] = np.float32(8.0)
    d["c5_logits"] = lg.reshape(-1)
    # config 5b: src0 storage [128,32,64,8] viewed as [128,64,32,8]; src1 [128,1,32,1]
    d["c5b_src0"] = normal(11, 128 * 32 * 64 * 8)
    d["c5b_src1"] = normal(12, 128 * 32)
    return d


def dense_nb(ne, elem=4):
    nb = [elem]
    for i in range(1, 4):
        nb.append(nb[-1] * ne[i - 1])
    return nb


# (name, config, algorithmic bytes, tensors) -- the byte counts are the
# minimum HBM traffic: every input read once and every output written once.
OPS = [
    ("add_broadcast_row", "config 1: f32 [4096,512] + [4096]", 8388608 + 16384 + 8388608),
    ("silu", "config 2: silu(gate) [11008,512]", 2 * 22544384),
    ("mul", "config 2: silu(gate) * up [11008,512]", 3 * 22544384),
    ("swiglu", "config 2: fused silu(gate) * up [11008,512]", 3 * 22544384),
    ("gelu", "config 2: gelu(gate) [11008,512]", 2 * 22544384),
    ("rms_norm", "config 3: rms_norm [4096,2048] eps=1e-5", 2 * 33554432),
    ("rms_norm_mul", "config 3: rms_norm * w [4096,2048], fused", 2 * 33554432 + 16384),
    ("soft_max_ext", "config 4: soft_max(x*scale + mask) [4096,512,32], f16 causal mask", 2 * 268435456 + 4194304),
    ("argmax_rows", "config 5: argmax per row [151936,64] -> i32", 38895616 + 256),
    ("sum_rows", "config 5: sum_rows [151936,64]", 38895616 + 256),
    ("mul_broadcast_4d", "config 5b: permuted [128,64,32,8] * [128,1,32,1]", 8388608 + 16384 + 8388608),
]
# Measured per op like the others but not part of the step (and so not of
# `value`): adjacent ops beyond the BASELINE configs' op list.
EXTRA_OPS = [
    ("glu_swiglu", "config 2 as one OpGlu (glu.rs): [up | gate] -> silu(gate) * up", 3 * 22544384),
    ("soft_max_dense", "OpSoftMax [4096,512], dense: f64 row sum (reductions.rs:565-601)", 2 * 8388608),
    ("soft_max_strided", "OpSoftMax [4096,512], rows 4 floats apart: exact sequential f32 row sum "
                         "(reductions.rs:603-638)", 2 * 8388608),
    ("generic_rms_norm", "config 3 through the generic envelope (GenericEvent RMS_NORM, generic.rs:1988-2055): "
                         "rms_norm [4096,2048] eps=1e-5, f64 scale", 2 * 33554432),
]
DOMINANT = "soft_max_ext"
COPY_BYTES = 2 * 268435456  # the calibration copy: 256 MiB read + 256 MiB written


ROTATE_BYTES = 1 << 30  # per-op timing cycles through at least this many distinct bytes
WARM_MS = 3.0  # each per-op graph (and copy reference) runs this long before it is timed


class GpuSuite:
    """Device buffers and the launch closures.

    Each op gets enough independent buffer sets that cycling through them
    moves at least ROTATE_BYTES (four times the 256 MB Infinity Cache), so
    back-to-back launches of one op stream from HBM, not from cache."""

    def __init__(self, host, stream, names):
        import torch

        import emel_hip as eh

        self.eh = eh
        self.torch = torch
        self.stream = stream
        self.kernel = eh.Kernel(stream=stream.cuda_stream, synchronous=False)
        dev = torch.device("cuda:0")
        L = eh.Layout
        F32, F16, I32 = eh.DType.F32, eh.DType.F16, eh.DType.I32

        def up(arr):
            return torch.from_numpy(arr).to(dev)

        def zeros(n, dtype=torch.float32):
            return torch.zeros(n, dtype=dtype, device=dev)

        def V(t, ne, nb=None, dtype=F32):
            return eh.TensorView(t, L(dtype, ne, nb or dense_nb(ne, 2 if dtype == F16 else 4)))

        def M(t, ne, nb=None, dtype=F32):
            return eh.TensorViewMut(t, L(dtype, ne, nb or dense_nb(ne)))

        silu_gate = np.empty_like(host["c2_gate"])  # mul's first operand: silu(gate) values
        silu_gate[:] = host["c2_gate"] / (1 + np.exp(-host["c2_gate"].astype(np.float64)))
        scale = float(np.float32(1.0 / np.sqrt(128.0)))
        snb = dense_nb([128, 32, 64, 8])
        vnb = [snb[0], snb[2], snb[1], snb[3]]  # dims 1 and 2 swapped
        n2 = 11008 * 512
        # name -> (host inputs, output (numel, dtype), event builder(inputs, output))
        spec = {
            "add_broadcast_row": ([host["c1_src0"], host["c1_src1"]], (4096 * 512, torch.float32),
                                  lambda i, o: eh.OpAddBroadcastRow(V(i[0], [4096, 512, 1, 1]), V(i[1], [4096, 1, 1, 1]),
                                                                    M(o, [4096, 512, 1, 1]))),
            "silu": ([host["c2_gate"]], (n2, torch.float32),
                     lambda i, o: eh.OpSilu(V(i[0], [11008, 512, 1, 1]), M(o, [11008, 512, 1, 1]))),
            "gelu": ([host["c2_gate"]], (n2, torch.float32),
                     lambda i, o: eh.OpGelu(V(i[0], [11008, 512, 1, 1]), M(o, [11008, 512, 1, 1]))),
            "mul": ([silu_gate, host["c2_up"]], (n2, torch.float32),
                    lambda i, o: eh.OpMul(V(i[0], [11008, 512, 1, 1]), V(i[1], [11008, 512, 1, 1]),
                                          M(o, [11008, 512, 1, 1]))),
            "swiglu": ([host["c2_gate"], host["c2_up"]], (n2, torch.float32),
                       lambda i, o: eh.OpSwiglu(V(i[0], [11008, 512, 1, 1]), V(i[1], [11008, 512, 1, 1]),
                                                M(o, [11008, 512, 1, 1]))),
            "rms_norm": ([host["c3_x"]], (4096 * 2048, torch.float32),
                         lambda i, o: eh.OpRmsNorm(V(i[0], [4096, 2048, 1, 1]), M(o, [4096, 2048, 1, 1]), 1e-5)),
            "rms_norm_mul": ([host["c3_x"], host["c3_w"]], (4096 * 2048, torch.float32),
                             lambda i, o: eh.OpRmsNormMul(V(i[0], [4096, 2048, 1, 1]), V(i[1], [4096, 1, 1, 1]),
                                                          M(o, [4096, 2048, 1, 1]), 1e-5)),
            "soft_max_ext": ([host["c4_x"], host["c4_mask"]], (4096 * 512 * 32, torch.float32),
                             lambda i, o: eh.OpSoftMaxExt(V(i[0], [4096, 512, 32, 1]),
                                                          V(i[1], [4096, 512, 1, 1], dtype=F16), scale,
                                                          M(o, [4096, 512, 32, 1]))),
            "argmax_rows": ([host["c5_logits"]], (64, torch.int32),
                            lambda i, o: eh.OpArgmaxRows(V(i[0], [151936, 64, 1, 1]), M(o, [1, 64, 1, 1], dtype=I32))),
            "sum_rows": ([host["c5_logits"]], (64, torch.float32),
                         lambda i, o: eh.OpSumRows(V(i[0], [151936, 64, 1, 1]), M(o, [1, 64, 1, 1]))),
            "mul_broadcast_4d": ([host["c5b_src0"], host["c5b_src1"]], (128 * 64 * 32 * 8, torch.float32),
                                 lambda i, o: eh.OpBinaryBroadcast(eh.BinaryOp.MUL, V(i[0], [128, 64, 32, 8], vnb),
                                                                   V(i[1], [128, 1, 32, 1]), M(o, [128, 64, 32, 8]))),
            "soft_max_dense": ([host["c1_src0"] * np.float32(4)], (4096 * 512, torch.float32),
                               lambda i, o: eh.OpSoftMax(V(i[0], [4096, 512, 1, 1]), M(o, [4096, 512, 1, 1]))),
            "soft_max_strided": ([np.pad((host["c1_src0"] * np.float32(4)).reshape(512, 4096), ((0, 0), (0, 4)))
                                  .reshape(-1)], (4096 * 512, torch.float32),
                                 lambda i, o: eh.OpSoftMax(V(i[0], [4096, 512, 1, 1], [4, 4 * 4100, 4 * 4100 * 512,
                                                                                        4 * 4100 * 512]),
                                                           M(o, [4096, 512, 1, 1]))),
            "glu_swiglu": ([np.concatenate([host["c2_up"], host["c2_gate"]])], (n2, torch.float32),
                           lambda i, o: eh.OpGlu(i[0], o, eh.GluSubOp.SWIGLU)),
            "generic_rms_norm": ([host["c3_x"]], (4096 * 2048, torch.float32),
                                 lambda i, o: eh.GenericEvent(eh.GenericRequest(
                                     eh.GenericOp.RMS_NORM, V(i[0], [4096, 2048, 1, 1]), None, None,
                                     M(o, [4096, 2048, 1, 1]), eh.OpParams(np.float32(1e-5).tobytes(), 4)))),
            "copy": ([np.zeros(COPY_BYTES // 8, np.float32)], (COPY_BYTES // 8, torch.float32),
                     lambda i, o: eh.OpScale(V(i[0], [COPY_BYTES // 8, 1, 1, 1]), M(o, [COPY_BYTES // 8, 1, 1, 1]),
                                             1.0)),
        }
        self.events = {}
        self.outputs = {}
        self.copies = {}
        for name in names:
            if name not in spec:
                raise ValueError(name)
            inputs, (numel, odt), build = spec[name]
            alg = dict((n, b) for n, _, b in OPS + EXTRA_OPS).get(name, COPY_BYTES)
            copies = max(2, -(-ROTATE_BYTES // alg))
            first = [up(x) for x in inputs]
            evs, outs = [], []
            for c in range(copies):
                ins = first if c == 0 else [t.clone() for t in first]
                o = zeros(numel, odt)
                evs.append(build(ins, o))
                outs.append(o)
            self.events[name] = evs
            self.outputs[name] = outs
            self.copies[name] = copies
        torch.cuda.synchronize()

    def launch(self, name, step):
        st = self.kernel.process_event(self.events[name][step % len(self.events[name])])
        if st != self.eh.Status.OK:
            raise RuntimeError(f"{name}: {st.name}: {self.eh.last_error()}")


COPY_SHAPES = ("FLAT", "WAVE4", "WAVE8", "WALK")


def copy_ceilings(suite, sizes, steps, capture, timed, warm):
    """Times a bit copy moving each algorithmic byte count (half read, half
    written) with every streaming shape of emel_stream_copy (one float4 per
    thread; 4 or 8 float4 per lane, wave-contiguous; one resident generation
    walking grid-stride), over rotating buffer sets totalling >=
    ROTATE_BYTES.  Returns {bytes: {shape: ms per launch}}."""
    torch, eh = suite.torch, suite.eh
    sid = suite.stream.cuda_stream
    out = {}
    for nbytes in sorted(set(sizes)):
        n = (nbytes // 8) // 64 * 64  # floats per side, 256-byte aligned slices
        slots = max(2, -(-ROTATE_BYTES // (8 * n)))
        src = torch.zeros(slots * n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty(slots * n, dtype=torch.float32, device="cuda:0")
        s0, d0 = src.data_ptr(), dst.data_ptr()
        res = {}
        for shape_name in COPY_SHAPES:
            shape = eh.CopyShape[shape_name]

            def launch(i, shape=shape):
                k = i % slots
                st = eh.stream_copy(s0 + 4 * n * k, d0 + 4 * n * k, 4 * n, shape, sid)
                if st != eh.Status.OK:
                    raise RuntimeError(f"copy {shape.name}: {st.name}: {eh.last_error()}")

            for i in range(2):
                launch(i)
            reps = max(steps, 20, slots)
            g = capture(lambda reps=reps, launch=launch: [launch(i) for i in range(reps)])
            warm(g)
            res[shape_name] = timed(lambda i: g.replay(), 3) / (3 * reps) * (nbytes / (8.0 * n))
            del g
        out[nbytes] = res
        del src, dst
    return out


def pcie_inclusive(suite, host, stream, reps=5):
    """soft_max_ext for a caller whose tensors live in (pinned) host memory:
    copy the scores and mask in, run the op, copy the result out, all on the
    kernel stream.  Returns the median time and the algorithmic bytes / time
    rate; this is never bench's `value`."""
    torch, eh = suite.torch, suite.eh
    x_h = torch.from_numpy(host["c4_x"]).pin_memory()
    m_h = torch.from_numpy(host["c4_mask"].view(np.float16)).pin_memory()
    y_h = torch.empty(x_h.numel(), dtype=torch.float32).pin_memory()
    x_d = torch.empty(x_h.numel(), dtype=torch.float32, device="cuda:0")
    m_d = torch.empty(m_h.numel(), dtype=torch.float16, device="cuda:0")
    y_d = torch.empty_like(x_d)
    F32, F16 = eh.DType.F32, eh.DType.F16
    ev = eh.OpSoftMaxExt(eh.TensorView(x_d, eh.Layout(F32, [4096, 512, 32, 1], dense_nb([4096, 512, 32, 1]))),
                         eh.TensorView(m_d, eh.Layout(F16, [4096, 512, 1, 1], dense_nb([4096, 512, 1, 1], 2))),
                         float(np.float32(1.0 / np.sqrt(128.0))),
                         eh.TensorViewMut(y_d, eh.Layout(F32, [4096, 512, 32, 1], dense_nb([4096, 512, 32, 1]))))
    times = []
    with torch.cuda.stream(stream):
        for _ in range(reps + 1):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            x_d.copy_(x_h, non_blocking=True)
            m_d.copy_(m_h, non_blocking=True)
            st = suite.kernel.process_event(ev)
            if st != eh.Status.OK:
                raise RuntimeError(f"soft_max_ext: {st.name}")
            y_h.copy_(y_d, non_blocking=True)
            b.record(stream)
            b.synchronize()
            times.append(a.elapsed_time(b))
    ms = float(np.median(times[1:]))
    nbytes = dict((n, b) for n, _, b in OPS)["soft_max_ext"]
    return {"op": "soft_max_ext", "ms": round(ms, 3), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "note": "inputs copied in from and the output copied out to pinned host memory around each launch"}


GATHER_VOCAB, GATHER_DIM, GATHER_TOKENS = 32000, 4096, 512
# format -> (dtype code, bytes per source row, event class name)
GATHER_FORMATS = {
    "f32": (0, GATHER_DIM * 4, "OpGetRows"),
    "f16": (1, GATHER_DIM * 2, "OpGetRowsF16"),
    "bf16": (30, GATHER_DIM * 2, "OpGetRowsBf16"),
    "q8_0": (8, GATHER_DIM // 32 * 34, "OpGetRowsQ8_0"),
    "q4_0": (2, GATHER_DIM // 32 * 18, "OpGetRowsQ4_0"),
    "q4_k": (12, GATHER_DIM // 256 * 144, "OpGetRowsQ4K"),
}


def gather_ops(suite, stream, reps):
    """Embedding lookups (get_rows.rs): GATHER_TOKENS ids into a
    [GATHER_DIM, GATHER_VOCAB] table of each source format, f32 output.
    call_us: one call between HIP events with device-resident ids (the
    index guard copies them to the host and waits); call_us_host_ids: the
    same with host-resident ids (checked in place, passed by value);
    kernel_us: a captured graph of back-to-back host-id calls cycling through
    table / output / id copies totalling >= ROTATE_BYTES, so rows come from
    HBM as in a decode step whose other layers flushed the caches."""
    torch, eh = suite.torch, suite.eh
    g = rng(21)
    dne = [GATHER_DIM, GATHER_TOKENS, 1, 1]
    sne = [GATHER_DIM, GATHER_VOCAB, 1, 1]
    res = {}
    for fmt, (code, row_bytes, cls) in GATHER_FORMATS.items():
        table_bytes = row_bytes * GATHER_VOCAB
        out_bytes = GATHER_DIM * GATHER_TOKENS * 4
        copies = max(2, -(-ROTATE_BYTES // (table_bytes + out_bytes)))
        evs_host, keep = [], []
        ev_dev = None
        for c in range(copies):
            if code == 0:
                table = torch.randn(GATHER_DIM * GATHER_VOCAB, device="cuda:0")
                lay = eh.Layout(code, sne, dense_nb(sne))
            elif code in (1, 30):
                table = torch.randn(GATHER_DIM * GATHER_VOCAB, device="cuda:0").to(
                    torch.float16 if code == 1 else torch.bfloat16)
                lay = eh.Layout(code, sne, dense_nb(sne, 2))
            else:
                raw = torch.randint(0, 256, (table_bytes,), dtype=torch.uint8, device="cuda:0")
                per_block = 144 if code == 12 else (34 if code == 8 else 18)
                blocks = raw.view(-1, per_block)
                hdr = 4 if code == 12 else 2
                scales = (torch.rand(blocks.shape[0] * hdr // 2, device="cuda:0") * 0.01).to(torch.float16)
                blocks[:, :hdr] = scales.view(torch.uint8).view(-1, hdr)
                table = raw
                lay = eh.Layout.packed(code, sne)
            out = torch.empty(GATHER_DIM * GATHER_TOKENS, dtype=torch.float32, device="cuda:0")
            ids_host = g.integers(0, GATHER_VOCAB, GATHER_TOKENS).astype(np.int32)
            dst = eh.TensorViewMut(out, eh.Layout(eh.DType.F32, dne, dense_nb(dne)))
            evs_host.append(getattr(eh, cls)(eh.TensorView(table, lay), eh.IndexView(ids_host, [GATHER_TOKENS, 1, 1]),
                                             dst))
            if c == 0:
                ids_dev = torch.from_numpy(ids_host).to("cuda:0")
                ev_dev = getattr(eh, cls)(eh.TensorView(table, lay), eh.IndexView(ids_dev, [GATHER_TOKENS, 1, 1]),
                                          dst)
                keep.append(ids_dev)
            keep += [table, out, ids_host]

        def call(e):
            st = suite.kernel.process_event(e)
            if st != eh.Status.OK:
                raise RuntimeError(f"get_rows {fmt}: {st.name}: {eh.last_error()}")

        def per_call(e):
            times = []
            with torch.cuda.stream(stream):
                for i in range(reps + 2):
                    a = torch.cuda.Event(enable_timing=True)
                    b = torch.cuda.Event(enable_timing=True)
                    a.record(stream)
                    call(e)
                    b.record(stream)
                    b.synchronize()
                    if i >= 2:
                        times.append(a.elapsed_time(b))
            return float(np.median(times)) * 1e3

        us = per_call(ev_dev)
        us_host = per_call(evs_host[0])
        n = max(reps, copies)
        with torch.cuda.stream(stream):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=stream):
                for i in range(n):
                    call(evs_host[i % copies])
            stream.synchronize()
            gr.replay()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(3):
                gr.replay()
            b.record(stream)
            b.synchronize()
            kus = a.elapsed_time(b) * 1e3 / (3 * n)
        alg = GATHER_TOKENS * (row_bytes + GATHER_DIM * 4 + 4)
        res[f"get_rows_{fmt}"] = {"config": f"{GATHER_TOKENS} ids into a [{GATHER_DIM},{GATHER_VOCAB}] {fmt} table",
                                  "alg_bytes": alg, "call_us": round(us, 2), "call_us_host_ids": round(us_host, 2),
                                  "kernel_us": round(kus, 3), "GB/s": round(alg / (kus * 1e-6) / 1e9, 1),
                                  "frac_of_peak": round(alg / (kus * 1e-6) / 1e9 / PEAK_GBS, 4),
                                  "rotation": f"{copies} table/output/id copies"}
        del gr, evs_host, ev_dev, keep
        torch.cuda.empty_cache()
    return res


SAMPLER_VOCAB, SAMPLER_ROWS = 151936, 64
SAMPLER_CASES = [(0.8, 40), (1.0, 8192)]  # (temperature, top_k)


def sampler_ops(suite, stream, reps):
    """emel-logits' native temperature/top-k sampler (sampler/sm.rs) over
    config 5's logits: SAMPLER_ROWS sequences of a SAMPLER_VOCAB vocabulary,
    N(0,1), sampled in one batched call.  The call rewrites the logits in
    place (they end as probabilities), so every timed call reads a fresh
    copy: kernel_us comes from back-to-back eager calls over `copies` buffers
    refreshed before each series, outside the timing (the sampler refuses
    graph capture: its random_state advances on the host).
    alg_bytes: logits read once and probabilities written once (the outputs
    per row are a few hundred bytes).  The CPU side is timed in
    cpu_baseline (sampler_rows_per_s)."""
    torch, eh = suite.torch, suite.eh
    import ctypes

    from emel_hip.abi import CSampleRows

    lib = eh.load()
    g = rng(31)
    card, rows = SAMPLER_VOCAB, SAMPLER_ROWS
    host = g.standard_normal((rows, card), dtype=np.float64).astype(np.float32)
    pristine = torch.from_numpy(host.reshape(-1)).to("cuda:0")
    alg = 2 * rows * card * 4
    copies = max(2, -(-ROTATE_BYTES // (rows * card * 4)))
    res = {}
    for temperature, top_k in SAMPLER_CASES:
        bufs = [pristine.clone() for _ in range(copies)]
        srt = torch.empty(rows * card, dtype=torch.int32, device="cuda:0")
        tp = torch.empty(rows * top_k, device="cuda:0")
        ti = torch.empty(rows * top_k, dtype=torch.int32, device="cuda:0")
        sel = torch.empty(rows, dtype=torch.int32, device="cuda:0")
        sc = torch.empty(rows, device="cuda:0")
        states = np.array(g.integers(1, 2147483647, rows), np.uint32)
        cr = CSampleRows(rows, card, card, top_k)
        reqs = [eh.SampleTemperatureTopK(card, temperature, top_k, b, srt, tp, ti, states, sel, sc).c() for b in bufs]

        def call(i):
            st = lib.emel_sample_temperature_top_k_rows(ctypes.byref(reqs[i % copies]), ctypes.byref(cr),
                                                        ctypes.c_void_p(stream.cuda_stream))
            if st != 0:
                raise RuntimeError(f"sampler: {eh.Status(st).name}: {eh.last_error()}")

        def refresh():
            for b in bufs:
                b.copy_(pristine)

        with torch.cuda.stream(stream):
            refresh()
            times = []
            for i in range(reps + 2):
                refresh()
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(stream)
                call(0)
                b.record(stream)
                b.synchronize()
                if i >= 2:
                    times.append(a.elapsed_time(b))
            call_us = float(np.median(times)) * 1e3
            # back-to-back eager calls (the sampler is not capturable: its
            # random_state advances on the host); the host enqueues ahead of
            # the device, so the span between the events is device time
            ktimes = []
            for _ in range(3):
                refresh()
                stream.synchronize()
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(stream)
                for i in range(copies):
                    call(i)
                b.record(stream)
                b.synchronize()
                ktimes.append(a.elapsed_time(b) * 1e3 / copies)
            kus = float(np.median(ktimes))
        res[f"sample_t{temperature}_k{top_k}"] = {
            "config": f"{rows} rows x {card} logits, temperature {temperature}, top_k {top_k}",
            "alg_bytes": alg, "call_us": round(call_us, 2), "kernel_us": round(kus, 2),
            "GB/s": round(alg / (kus * 1e-6) / 1e9, 1), "frac_of_peak": round(alg / (kus * 1e-6) / 1e9 / PEAK_GBS, 4),
            "rows_per_s": round(rows / (kus * 1e-6), 1),
            "rotation": f"{copies} logits copies refreshed before each replay"}
        del bufs, reqs
        torch.cuda.empty_cache()
    return res


def cpu_baseline(host, runs=5, op_budget_s=30.0):
    """The C oracle (a single-threaded restatement of the reference's CPU
    path: view decode, glibc libm) on the exact config tensors, the same
    host bytes bench uploads: per op one warm-up run, then `runs` timed runs
    (the reference's own policy, snapshots/bench/kernel-elementwise-aarch64.txt:8),
    median, monotonic clock.  An op whose runs pass op_budget_s stops early
    and reports how many it took.  Returns (GB/s over all ops, per op,
    sampler)."""
    import oracle as orc

    def v(a, ne, nb=None, dtype=None):
        return orc.view(a, ne, nb, dtype)

    n2 = 11008 * 512
    g, u = host["c2_gate"], host["c2_up"]
    x3, x4, x5 = host["c3_x"], host["c4_x"], host["c5_logits"]
    scale = float(np.float32(1.0 / np.sqrt(128.0)))
    snb = dense_nb([128, 32, 64, 8])
    vnb = [snb[0], snb[2], snb[1], snb[3]]
    outs = {"c1": np.zeros(4096 * 512, np.float32), "c2": np.zeros(n2, np.float32),
            "c3": np.zeros(4096 * 2048, np.float32), "c4": np.zeros(4096 * 512 * 32, np.float32),
            "c5i": np.zeros(64, np.int32), "c5f": np.zeros(64, np.float32), "c5b": np.zeros(128 * 64 * 32 * 8, np.float32)}
    calls = {
        "add_broadcast_row": lambda: orc.broadcast_row(orc.ADD, v(host["c1_src0"], [4096, 512, 1, 1]),
                                                       v(host["c1_src1"], [4096, 1, 1, 1]), v(outs["c1"], [4096, 512, 1, 1])),
        "silu": lambda: orc.unary_event(10, v(g, [11008, 512, 1, 1]), v(outs["c2"], [11008, 512, 1, 1])),
        "mul": lambda: orc.binary(orc.MUL, v(g, [11008, 512, 1, 1]), v(u, [11008, 512, 1, 1]),
                                  v(outs["c2"], [11008, 512, 1, 1])),
        "swiglu": lambda: orc.swiglu(v(g, [11008, 512, 1, 1]), v(u, [11008, 512, 1, 1]), v(outs["c2"], [11008, 512, 1, 1])),
        "gelu": lambda: orc.unary_event(8, v(g, [11008, 512, 1, 1]), v(outs["c2"], [11008, 512, 1, 1])),
        "rms_norm": lambda: orc.rms_norm(v(x3, [4096, 2048, 1, 1]), v(outs["c3"], [4096, 2048, 1, 1]), 1e-5),
        "rms_norm_mul": lambda: orc.rms_norm_mul(v(x3, [4096, 2048, 1, 1]), v(host["c3_w"], [4096, 1, 1, 1]),
                                                 v(outs["c3"], [4096, 2048, 1, 1]), 1e-5),
        "soft_max_ext": lambda: orc.soft_max_ext(v(x4, [4096, 512, 32, 1]),
                                                 v(host["c4_mask"], [4096, 512, 1, 1], None, orc.F16), scale,
                                                 v(outs["c4"], [4096, 512, 32, 1])),
        "argmax_rows": lambda: orc.argmax_rows(v(x5, [151936, 64, 1, 1]), v(outs["c5i"], [1, 64, 1, 1])),
        "sum_rows": lambda: orc.sum_rows(v(x5, [151936, 64, 1, 1]), v(outs["c5f"], [1, 64, 1, 1])),
        "mul_broadcast_4d": lambda: orc.binary_bcast(orc.MUL, v(host["c5b_src0"], [128, 64, 32, 8], vnb),
                                                     v(host["c5b_src1"], [128, 1, 32, 1]), v(outs["c5b"], [128, 64, 32, 8])),
    }
    alg = dict((n, b) for n, _, b in OPS)

    def median_time(fn, what):
        st = fn()  # warm-up
        if st != orc.OK:
            raise RuntimeError(f"oracle {what} failed: {st}")
        times = []
        t_op = time.monotonic()
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
            if time.monotonic() - t_op > op_budget_s:
                break
        return float(np.median(times)), len(times)

    per_op = {}
    total_bytes = 0.0
    total_s = 0.0
    for name, fn in calls.items():
        t, n = median_time(fn, name)
        per_op[name] = {"GB/s": alg[name] / t / 1e9, "ns_per_op": t * 1e9, "runs": n}
        total_bytes += alg[name]
        total_s += t
    # the emel-logits sampler (not a step op): the oracle over the bench's
    # whole sampler workload (SAMPLER_ROWS rows), per SAMPLER_CASES entry
    sampler = {}
    rows = rng(31).standard_normal((SAMPLER_ROWS, SAMPLER_VOCAB), dtype=np.float64).astype(np.float32)
    for temperature, top_k in SAMPLER_CASES:
        def batch(temperature=temperature, top_k=top_k):
            for r in range(SAMPLER_ROWS):
                st = orc.sample_temperature_top_k(SAMPLER_VOCAB, temperature, top_k, rows[r].copy(),
                                                  np.zeros(SAMPLER_VOCAB, np.int32), np.zeros(top_k, np.float32),
                                                  np.zeros(top_k, np.int32), np.array([7], np.uint32),
                                                  np.zeros(1, np.int32), np.zeros(1, np.float32))
                if st != orc.OK:
                    return st
            return orc.OK

        t, n = median_time(batch, "sampler")
        sampler[f"sample_t{temperature}_k{top_k}"] = {"rows_per_s": round(SAMPLER_ROWS / t, 2),
                                                      "GB/s": 2 * SAMPLER_ROWS * SAMPLER_VOCAB * 4 / t / 1e9,
                                                      "ns_per_op": t * 1e9, "runs": n}
    return total_bytes / total_s / 1e9, per_op, sampler


def profile_launches(host, stream, names, count):
    """Eager launches only, for counter collection: each op `count` times on
    rotating buffer sets (cold data), one op after another."""
    import torch

    suite = GpuSuite(host, stream, names)
    with torch.cuda.stream(stream):
        for n in names:
            for i in range(count):
                suite.launch(n, i)
            stream.synchronize()
            print(f"profile: {n} x{count}", flush=True)


def profile_sampler(host, stream, count):
    """Eager sampler calls for counter collection: each SAMPLER_CASES case
    `count` times over config 5's logits, a fresh copy per call."""
    import ctypes

    import torch

    from emel_hip.abi import CSampleRows

    suite = GpuSuite(host, stream, [])
    eh = suite.eh
    lib = eh.load()
    g = rng(31)
    card, rows = SAMPLER_VOCAB, SAMPLER_ROWS
    pristine = torch.from_numpy(g.standard_normal((rows, card), dtype=np.float64).astype(np.float32).reshape(-1)).to(
        "cuda:0")
    with torch.cuda.stream(stream):
        for temperature, top_k in SAMPLER_CASES:
            buf = pristine.clone()
            srt = torch.empty(rows * card, dtype=torch.int32, device="cuda:0")
            tp = torch.empty(rows * top_k, device="cuda:0")
            ti = torch.empty(rows * top_k, dtype=torch.int32, device="cuda:0")
            sel = torch.empty(rows, dtype=torch.int32, device="cuda:0")
            sc = torch.empty(rows, device="cuda:0")
            states = np.array(g.integers(1, 2147483647, rows), np.uint32)
            cr = CSampleRows(rows, card, card, top_k)
            req = eh.SampleTemperatureTopK(card, temperature, top_k, buf, srt, tp, ti, states, sel, sc).c()
            for _ in range(count):
                buf.copy_(pristine)
                st = lib.emel_sample_temperature_top_k_rows(ctypes.byref(req), ctypes.byref(cr),
                                                            ctypes.c_void_p(stream.cuda_stream))
                if st != 0:
                    raise RuntimeError(f"sampler: {eh.Status(st).name}: {eh.last_error()}")
            stream.synchronize()
            print(f"profile: sampler t{temperature} k{top_k} x{count}", flush=True)


def launch_floor(suite, capture, timed, reps=200):
    """Per-launch time of back-to-back dependent launches that do almost no
    work (OpScale over one float4), replayed from a graph: the fixed cost
    every launch pays before its bytes move."""
    torch, eh = suite.torch, suite.eh
    src = torch.zeros(4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty(4, dtype=torch.float32, device="cuda:0")
    lay = eh.Layout.contiguous(eh.DType.F32, [4, 1, 1, 1])
    ev = eh.OpScale(eh.TensorView(src, lay), eh.TensorViewMut(dst, lay), 1.0)

    def launch(i):
        if suite.kernel.process_event(ev) != eh.Status.OK:
            raise RuntimeError(f"launch floor: {eh.last_error()}")

    launch(0)
    g = capture(lambda: [launch(i) for i in range(reps)])
    g.replay()
    return timed(lambda i: g.replay(), 3) / (3 * reps) * 1e3


def host_facts():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return {"cpu": model, "nproc": os.cpu_count(), "affinity": affinity, "glibc": platform.libc_ver()[1]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ops", default="")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-copy", action="store_true", help="skip the same-size copy reference per op")
    ap.add_argument("--pcie", action="store_true", help="also time soft_max_ext with host-resident tensors")
    ap.add_argument("--no-gather", action="store_true", help="skip the get_rows embedding lookups")
    ap.add_argument("--no-sampler", action="store_true", help="skip the emel-logits sampler")
    ap.add_argument("--launches", type=int, default=0,
                    help="profiling mode: launch every selected op and the 256 MiB calibration copy this many times "
                         "(eagerly, cycling buffer sets), and each sampler case as often (unless --no-sampler or "
                         "--ops), then exit without timing; for rocprofv3 --pmc runs")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}): every op is row-local, "
              "so N GPUs would each run the same kernels on their own rows; no multi-GPU figure is measured", file=sys.stderr)
        sys.exit(2)

    import torch

    extra_names = [n for n, _, _ in EXTRA_OPS]
    names = [n for n, _, _ in OPS]
    extra = list(extra_names)
    if args.ops:
        wanted = [n for n in args.ops.split(",") if n]
        names = [n for n in wanted if n not in extra_names]
        extra = [n for n in wanted if n in extra_names]
    info = {n: (cfg, b) for n, cfg, b in OPS + EXTRA_OPS}
    info["copy"] = ("calibration copy: scale by 1.0 over 256 MiB", COPY_BYTES)

    host = config_inputs()
    stream = torch.cuda.Stream()
    if args.launches > 0:
        profile_launches(host, stream, names + extra + ["copy"], args.launches)
        if not args.no_sampler and not args.ops:
            profile_sampler(host, stream, args.launches)
        return
    suite = GpuSuite(host, stream, names + extra)

    with torch.cuda.stream(stream):
        for w in range(args.warmup):
            for n in names + extra:
                suite.launch(n, w)
        stream.synchronize()

        def timed(fn, reps):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for i in range(reps):
                fn(i)
            b.record(stream)
            b.synchronize()
            return a.elapsed_time(b)

        def capture(fn):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                fn()
            stream.synchronize()
            return g

        def warm(g):
            """Replays g for at least WARM_MS (and at least once)."""
            once = timed(lambda i: g.replay(), 1)
            for _ in range(int(WARM_MS / max(once, 1e-3))):
                g.replay()

        def two_steps():
            for c in range(2):
                for n in names:
                    suite.launch(n, c)

        # eager: K steps launched from the host, events only at the ends
        t0 = time.perf_counter()
        eager_step_ms = timed(lambda s: [suite.launch(n, s) for n in names], args.steps) / args.steps
        wall = time.perf_counter() - t0

        # graph: one capture of two steps (both buffer copies), replayed;
        # every replay must reproduce the eager outputs bit for bit
        step_graph = capture(two_steps)
        reference = {}
        for n in names:
            suite.launch(n, 0)
        stream.synchronize()
        for n in names:
            reference[n] = suite.outputs[n][0].clone()
        for check in range(2):
            for n in names:
                suite.outputs[n][0].zero_()
            stream.synchronize()
            step_graph.replay()
            stream.synchronize()
            for n in names:
                if not torch.equal(suite.outputs[n][0], reference[n]):
                    raise RuntimeError(f"graph replay {check} of {n} differs from the eager launch")
        pairs = max(1, args.steps // 2)
        step_ms = timed(lambda i: step_graph.replay(), pairs) / (2 * pairs)

        # per op: a graph of back-to-back launches cycling through all of
        # the op's buffer sets (>= ROTATE_BYTES), so each launch is cold.
        # The graph runs for WARM_MS before it is timed: an op timed right
        # after soft_max_ext's 541 MB launches ran ~1 us per launch slower for
        # about a millisecond (argmax_rows 11.2 against 9.9 us, sum_rows 10.0
        # against 9.1 us on one box), so each op is timed in its own steady
        # state.
        per_ms = {}
        for n in names + extra:
            reps = max(args.steps, 20, suite.copies[n])
            g = capture(lambda n=n, reps=reps: [suite.launch(n, i) for i in range(reps)])
            warm(g)
            per_ms[n] = timed(lambda i: g.replay(), 3) / (3 * reps)

        # same-size copy: a bit copy moving the op's algorithmic bytes with
        # each streaming shape, launched and rotated the same way; the fastest
        # is what a plain stream achieves at that size (launch ramp and tail
        # included)
        copy_ms = {}
        if not args.no_copy:
            copy_ms = copy_ceilings(suite, [info[n][1] for n in names + extra if n != "copy"], args.steps, capture,
                                    timed, warm)
        floor_us = launch_floor(suite, capture, timed)

    traffic = {}
    traffic_file = ROOT / "profiles" / "traffic.json"
    if traffic_file.exists():
        try:
            traffic = json.loads(traffic_file.read_text())
        except ValueError:
            traffic = {}

    def op_entry(n):
        cfg, nbytes = info[n]
        us = per_ms[n] * 1e3
        gbs = nbytes / (us * 1e-6) / 1e9
        e = {"config": cfg, "alg_bytes": nbytes, "us": round(us, 3), "GB/s": round(gbs, 1),
             "frac_of_peak": round(gbs / PEAK_GBS, 4)}
        if nbytes in copy_ms:
            shapes = copy_ms[nbytes]
            best = min(shapes, key=shapes.get)
            cus = shapes[best] * 1e3
            e["copy_us"] = round(cus, 3)
            e["copy_shape"] = best
            e["copy_us_by_shape"] = {k: round(v * 1e3, 3) for k, v in shapes.items()}
            e["frac_of_copy"] = round(cus / us, 4)
        t = traffic.get(n)
        if isinstance(t, dict) and "hbm_bytes_per_launch" in t:
            # rocprof FETCH_SIZE + WRITE_SIZE per launch (scaled by the calibration
            # copy), its ratio to the algorithmic bytes, and the rate at this time
            e["traffic"] = t["hbm_bytes_per_launch"]
            e["traffic_ratio"] = round(t["hbm_bytes_per_launch"] / nbytes, 4)
            e["traffic_GB/s"] = round(t["hbm_bytes_per_launch"] / (us * 1e-6) / 1e9, 1)
        return e

    per_op = {n: op_entry(n) for n in names}
    extra_ops = {n: op_entry(n) for n in extra}
    total_bytes = sum(info[n][1] for n in names)
    value = total_bytes / (step_ms * 1e-3) / 1e9

    measured = {**per_op, **extra_ops}
    dom = DOMINANT if DOMINANT in measured else (names + extra)[0]
    roof = {"kernel": dom, "bound": "hbm", "achieved": measured[dom]["GB/s"], "peak": PEAK_GBS, "unit": "GB/s",
            "frac": round(measured[dom]["GB/s"] / PEAK_GBS, 4), "traffic": None,
            "alg_bytes_per_launch": info[dom][1], "avg_launch_us": measured[dom]["us"]}
    t = traffic.get(dom)
    if isinstance(t, dict) and "hbm_bytes_per_launch" in t:
        roof["traffic"] = t["hbm_bytes_per_launch"]

    gather = None
    if not args.no_gather and not args.ops:
        gather = gather_ops(suite, stream, max(10, min(args.steps, 50)))

    sampler = None
    if not args.no_sampler and not args.ops:
        sampler = sampler_ops(suite, stream, max(5, min(args.steps, 20)))

    pcie = None
    if args.pcie and "soft_max_ext" in names:
        pcie = pcie_inclusive(suite, host, stream)

    cpu = None
    if not args.no_cpu and not args.ops:
        cpu_gbs, cpu_ops, cpu_sampler = cpu_baseline(host)
        facts = host_facts()
        cpu = {"value": round(cpu_gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": "C oracle (single-threaded restatement of the reference CPU path) on the exact config "
                         "tensors bench uploads: one warm-up run, then the median of 5 runs per op (fewer if an "
                         "op's runs pass 30 s; 'runs' says how many); value = all ops' algorithmic bytes / the sum "
                         "of their median times; sampler: all 64 rows of its workload",
               "host": facts,
               "per_op": {k: {"GB/s": round(v["GB/s"], 3), "ns_per_op": round(v["ns_per_op"]), "runs": v["runs"]}
                          for k, v in cpu_ops.items()},
               "sampler": {k: {"rows_per_s": v["rows_per_s"], "GB/s": round(v["GB/s"], 4),
                               "ns_per_op": round(v["ns_per_op"]), "runs": v["runs"]}
                           for k, v in cpu_sampler.items()}}

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded PCG64; BASELINE config shapes and distributions)",
        "config": {"workload": "all BASELINE configs, one launch of each op per step: " + ", ".join(names),
                   "launch": "one captured HIP graph of two steps replayed K/2 times (replays checked bit-exact "
                             "against eager launches); eager_ms_per_step: the same steps launched from Python",
                   "eager_ms_per_step": round(eager_step_ms, 4),
                   "buffer_policy": "step: >=1 GB of other ops moves between two launches of one op; per op (after 3 ms of warm-up replays): "
                                    "back-to-back launches cycle through >=1 GiB of distinct buffer sets "
                                    "(Infinity Cache is 256 MB)",
                   "wall_s": round(wall, 3),
                   "launch_floor_us": round(floor_us, 3)},
        "per_op": per_op,
        "extra_ops": extra_ops,
        "gather_ops": gather,
        "sampler_ops": sampler,
        "roofline": roof,
        "cpu_baseline": cpu,
        "pcie_inclusive": pcie,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
