"""Run by tests/test_gpu_graphs.py in a fresh process: which calls refuse a
stream under HIP graph capture, before anything is enqueued, and that the
refusal leaves the capture (and later eager calls) intact.

Fresh, because what is refused depends on per-process state: the first GELU
on a device and the first split reduction on a stream (scratch growth).  The
process's first call of the allocation-free argmax_rows is made under the
capture too: its one-time set-up (the scratch symbol's address, a fill
kernel on the stream) must be capturable, and the replay must match an eager
emel_op_argmax_rows.  Prints one JSON object of statuses."""
import ctypes
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "emel.rs_amd", ROOT / "tests"):
    sys.path.insert(0, str(p))

import numpy as np  # noqa: E402
import torch  # noqa: E402

import emel_hip as eh  # noqa: E402


def main():
    dev = torch.device("cuda:0")
    s = torch.cuda.Stream()
    k = eh.Kernel(stream=s.cuda_stream, synchronous=False)
    lay = eh.Layout.contiguous(eh.DType.F32, [4096, 64, 1, 1])
    g = torch.Generator(device="cpu").manual_seed(5)
    x = torch.randn(4096 * 64, generator=g).to(dev)
    y = torch.zeros_like(x)
    z = torch.zeros_like(x)
    total = torch.zeros(1, device=dev)
    ids_dev = torch.tensor([3, 1, 4], dtype=torch.int32, device=dev)
    gathered = torch.zeros(3 * 4096, device=dev)
    logits = torch.randn(1000, generator=g).to(dev)
    sorted_idx = torch.zeros(1000, dtype=torch.int32, device=dev)
    top_p = torch.zeros(8, device=dev)
    top_i = torch.zeros(8, dtype=torch.int32, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    score = torch.zeros(1, device=dev)
    state = np.array([777], np.uint32)
    tv, tm = eh.TensorView, eh.TensorViewMut
    one = eh.Layout.contiguous(eh.DType.F32, [1, 1, 1, 1])
    g_lay = eh.Layout.contiguous(eh.DType.F32, [4096, 3, 1, 1])
    i32_lay = eh.Layout(eh.DType.I32, [1, 64, 1, 1], [4, 4, 256, 256])
    am_graph = torch.full((64,), -1, dtype=torch.int32, device=dev)
    am_eager = torch.full((64,), -2, dtype=torch.int32, device=dev)
    lib = eh.load()
    torch.cuda.synchronize()
    # one eager call: the device check, not a GELU and not a reduction
    with torch.cuda.stream(s):
        assert k.process_event(eh.OpAdd(tv(x, lay), tv(x, lay), tm(z, lay))) == eh.Status.OK, eh.last_error()
    s.synchronize()
    want_add = (x + x).cpu()

    out = {}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out["gelu_first"] = int(k.process_event(eh.OpGelu(tv(x, lay), tm(y, lay))))
        out["sum_growth"] = int(k.process_event(eh.OpSum(tv(x, lay), tm(total, one))))
        out["l2_norm"] = int(k.process_event(eh.OpL2Norm(tv(x, lay), tm(y, lay))))
        out["get_rows_device_ids"] = int(k.process_event(
            eh.OpGetRows(tv(x, lay), eh.IndexView(ids_dev, [3, 1, 1]), tm(gathered, g_lay))))
        req = eh.SampleTemperatureTopK(1000, 0.7, 8, logits, sorted_idx, top_p, top_i, state, tok, score)
        out["sampler"] = int(eh.Sampler(stream=s.cuda_stream).sample_temperature_top_k(req)[0])
        out["add"] = int(k.process_event(eh.OpAdd(tv(x, lay), tv(x, lay), tm(z, lay))))
        # the process's first allocation-free call: set-up and launch captured
        out["argmax_no_alloc_first"] = int(lib.emel_op_argmax_rows_no_alloc(
            ctypes.byref(tv(x, lay).c()), ctypes.byref(tm(am_graph, i32_lay).c()), ctypes.c_void_p(s.cuda_stream)))
    out["state_unchanged"] = int(state[0]) == 777
    z.fill_(float("nan"))
    graph.replay()
    s.synchronize()
    out["replay_matches"] = bool(torch.equal(z.cpu(), want_add))
    with torch.cuda.stream(s):
        out["argmax_rows_eager"] = int(k.process_event(eh.OpArgmaxRows(tv(x, lay), tm(am_eager, i32_lay))))
    s.synchronize()
    out["argmax_no_alloc_matches"] = bool(torch.equal(am_graph.cpu(), am_eager.cpu()))
    am_graph.fill_(-1)  # a second replay after other work on the stream
    graph.replay()
    s.synchronize()
    out["argmax_no_alloc_replay2"] = bool(torch.equal(am_graph.cpu(), am_eager.cpu()))
    # after the capture every refused call runs eagerly
    with torch.cuda.stream(s):
        out["gelu_eager"] = int(k.process_event(eh.OpGelu(tv(x, lay), tm(y, lay))))
        out["sum_eager"] = int(k.process_event(eh.OpSum(tv(x, lay), tm(total, one))))
        out["l2_norm_eager"] = int(k.process_event(eh.OpL2Norm(tv(x, lay), tm(y, lay))))
        out["get_rows_eager"] = int(k.process_event(
            eh.OpGetRows(tv(x, lay), eh.IndexView(ids_dev, [3, 1, 1]), tm(gathered, g_lay))))
    s.synchronize()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
