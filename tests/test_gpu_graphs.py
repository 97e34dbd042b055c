"""GPU: HIP graph capture of the library's calls.

1. A step of capturable calls (elementwise, broadcast, rows, reductions,
   strided soft_max, get_rows with host ids, the generic envelope, the
   allocation-free argmax_rows) is run eagerly, captured once and replayed
   three times.  Before each replay the outputs are overwritten with NaN and
   an unrelated eager call runs on the same stream; every replay must
   reproduce the eager outputs bit for bit.
2. In a fresh process (tests/graph_capture_child.py), the calls that would
   allocate, wait or advance host state refuse a capturing stream with
   EMEL_ERR_STREAM_CAPTURE before enqueuing anything; the capture stays
   valid, and the same calls succeed eagerly afterwards.  The process's
   first allocation-free argmax_rows call is made under that capture and
   its replays match an eager emel_op_argmax_rows.
"""
import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import emel_hip as eh
from helpers import normal

pytestmark = pytest.mark.gpu

CHILD = Path(__file__).resolve().parent / "graph_capture_child.py"


def test_captured_step_replays_bit_exact(gpu):
    import ctypes

    import torch

    lib = eh.load()

    s = torch.cuda.Stream()
    k = eh.Kernel(stream=s.cuda_stream, synchronous=False)
    F32 = eh.DType.F32
    cols, rows = 4096, 64
    lay = eh.Layout.contiguous(F32, [cols, rows, 1, 1])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    x = t(normal(901, cols * rows, 2.0))
    x2 = t(normal(902, cols * rows))
    w = t(normal(903, cols))
    mask = t(np.where(np.random.Generator(np.random.PCG64(904)).random(cols * rows) < 0.2, -np.inf, 0.0)
             .astype(np.float16))
    padded = t(normal(905, (cols + 4) * rows, 3.0))
    other = t(normal(906, cols * rows))
    ids = np.array([5, 0, 63, 17], np.int32)
    outs = {name: torch.zeros(cols * rows, device=gpu) for name in
            ("add", "rms_mul", "smx_ext", "swiglu", "strided", "generic_rms", "sigmoid", "group", "clamp", "gelu")}
    outs["sum_rows"] = torch.zeros(rows, device=gpu)
    outs["argmax"] = torch.zeros(rows, dtype=torch.int32, device=gpu)
    outs["argmax_na"] = torch.zeros(rows, dtype=torch.int32, device=gpu)
    outs["rows"] = torch.zeros(len(ids) * cols, device=gpu)
    scratch_out = torch.zeros(rows, device=gpu)
    tv, tm = eh.TensorView, eh.TensorViewMut
    row_lay = eh.Layout.contiguous(F32, [1, rows, 1, 1])
    i32_lay = eh.Layout(eh.DType.I32, [1, rows, 1, 1], [4, 4, 4 * rows, 4 * rows])
    pad_lay = eh.Layout(F32, [cols, rows, 1, 1], [4, 4 * (cols + 4), 4 * (cols + 4) * rows, 4 * (cols + 4) * rows])
    mask_lay = eh.Layout.dense(eh.DType.F16, [cols, rows, 1, 1])
    get_lay = eh.Layout.contiguous(F32, [cols, len(ids), 1, 1])
    group_lay = eh.Layout.contiguous(F32, [64, 64, 64, 1])

    def step():
        ev = [
            eh.OpAdd(tv(x, lay), tv(x2, lay), tm(outs["add"], lay)),
            eh.OpRmsNormMul(tv(x, lay), tv(w, eh.Layout.contiguous(F32, [cols, 1, 1, 1])), tm(outs["rms_mul"], lay),
                            1e-6),
            eh.OpSoftMaxExt(tv(x, lay), tv(mask, mask_lay), 0.125, tm(outs["smx_ext"], lay)),
            eh.OpSwiglu(tv(x, lay), tv(x2, lay), tm(outs["swiglu"], lay)),
            eh.OpSoftMax(tv(padded, pad_lay), tm(outs["strided"], lay)),
            eh.OpSumRows(tv(x, lay), tm(outs["sum_rows"], row_lay)),
            eh.OpArgmaxRows(tv(x, lay), tm(outs["argmax"], i32_lay)),
            eh.OpSigmoid(tv(x, lay), tm(outs["sigmoid"], lay)),
            eh.OpGroupNorm(tv(x, group_lay), tm(outs["group"], group_lay), 8, 1e-5),
            eh.OpClamp(tv(x, lay), tm(outs["clamp"], lay), -0.5, 0.75),
            eh.OpGelu(tv(x, lay), tm(outs["gelu"], lay)),
            eh.OpGetRows(tv(x, lay), eh.IndexView(ids, [len(ids), 1, 1]), tm(outs["rows"], get_lay)),
            eh.GenericEvent(eh.GenericRequest(eh.GenericOp.RMS_NORM, tv(x2, lay), None, None,
                                              tm(outs["generic_rms"], lay), eh.OpParams.f32(1e-5))),
        ]
        for e in ev:
            assert k.process_event(e) == eh.Status.OK, (type(e).__name__, eh.last_error())
        st = lib.emel_op_argmax_rows_no_alloc(ctypes.byref(tv(x, lay).c()), ctypes.byref(tm(outs["argmax_na"],
                                              i32_lay).c()), s.cuda_stream)
        assert st == int(eh.Status.OK), eh.last_error()

    with torch.cuda.stream(s):
        step()
    s.synchronize()
    eager = {name: o.cpu().clone() for name, o in outs.items()}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step()
    for rep in range(3):
        with torch.cuda.stream(s):
            for o in outs.values():
                o.fill_(-1 if o.dtype == torch.int32 else float("nan"))
            # unrelated eager work on the same stream between replays
            assert k.process_event(eh.OpSumRows(tv(other, lay), tm(scratch_out, row_lay))) == eh.Status.OK
            graph.replay()  # on s, after that call: they share the stream's scratch
        s.synchronize()
        for name, o in outs.items():
            got = o.cpu()
            assert torch.equal(got.view(torch.int32), eager[name].view(torch.int32)), (rep, name)


def test_refusals_under_capture_in_a_fresh_process(gpu):
    print("child:", CHILD.name, flush=True)
    r = subprocess.run([sys.executable, str(CHILD)], capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-3000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    cap = int(eh.Status.STREAM_CAPTURE)
    for key in ("gelu_first", "sum_growth", "l2_norm", "get_rows_device_ids", "sampler"):
        assert out[key] == cap, (key, out)
    assert out["add"] == int(eh.Status.OK), out
    assert out["state_unchanged"] and out["replay_matches"], out
    # the first allocation-free call of the process, made under capture
    assert out["argmax_no_alloc_first"] == int(eh.Status.OK), out
    assert out["argmax_rows_eager"] == int(eh.Status.OK), out
    assert out["argmax_no_alloc_matches"] and out["argmax_no_alloc_replay2"], out
    for key in ("gelu_eager", "sum_eager", "l2_norm_eager", "get_rows_eager"):
        assert out[key] == int(eh.Status.OK), (key, out)


RESERVE_CHILD = Path(__file__).resolve().parent / "reserve_capture_child.py"


def test_reserved_scratch_and_prepared_tables_allow_capture(gpu):
    """emel_stream_reserve and emel_device_prepare, in a fresh process: the
    first GELU and the first split reductions on the stream are captured
    (without them they are refused, as the test above shows), replays equal
    eager calls, and the reserved sizes are what the stream holds."""
    print("child:", RESERVE_CHILD.name, flush=True)
    r = subprocess.run([sys.executable, str(RESERVE_CHILD)], capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-3000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    ok, cap = int(eh.Status.OK), int(eh.Status.STREAM_CAPTURE)
    assert out["workspace_before"] == [ok, 0, 0], out
    assert out["prepare"] == ok and out["reserve"] == ok, out
    st, work, counters = out["workspace_after"]
    assert st == ok and work >= 4 << 20 and counters >= 1 << 20, out
    assert out["captured"] == [ok, ok, ok], out
    assert out["reserve_under_capture"] == cap, out
    assert out["eager"] == [ok, ok, ok], out
    assert all(out["replay_matches"].values()) and all(out["replay2_matches"].values()), out
    assert out["workspace_end"] == out["workspace_after"], out
