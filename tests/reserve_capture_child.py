"""Run by tests/test_gpu_graphs.py in a fresh process: with the stream's
scratch reserved (emel_stream_reserve) and the device's tables built
(emel_device_prepare) up front, the process's first GELU and first split
reductions on the stream run under HIP graph capture instead of being
refused, and every replay equals eager calls of the same ops.  Also that
reserving under capture is refused and leaves the capture intact.  Prints
one JSON object."""
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "emel.rs_amd", ROOT / "tests"):
    sys.path.insert(0, str(p))

import torch  # noqa: E402

import emel_hip as eh  # noqa: E402


def main():
    dev = torch.device("cuda:0")
    s = torch.cuda.Stream()
    sid = s.cuda_stream
    k = eh.Kernel(stream=sid, synchronous=False)
    tv, tm = eh.TensorView, eh.TensorViewMut
    rows, cols = 64, 151936
    lay = eh.Layout.contiguous(eh.DType.F32, [cols, rows, 1, 1])
    row_out = eh.Layout.contiguous(eh.DType.F32, [1, rows, 1, 1])
    i32_lay = eh.Layout(eh.DType.I32, [1, rows, 1, 1], [4, 4, 4 * rows, 4 * rows])
    g = torch.Generator(device="cpu").manual_seed(9)
    x = torch.randn(rows * cols, generator=g).to(dev)
    outs = {"gelu": torch.zeros_like(x), "sum_rows": torch.zeros(rows, device=dev),
            "argmax_rows": torch.zeros(rows, dtype=torch.int32, device=dev)}
    torch.cuda.synchronize()
    out = {}
    st, w0, c0 = eh.stream_workspace(sid)
    out["workspace_before"] = [int(st), w0, c0]
    out["prepare"] = int(eh.device_prepare(sid))
    out["reserve"] = int(eh.stream_reserve(4 << 20, 1 << 20, sid))
    st, w1, c1 = eh.stream_workspace(sid)
    out["workspace_after"] = [int(st), w1, c1]

    def step():
        r = [int(k.process_event(eh.OpGelu(tv(x, lay), tm(outs["gelu"], lay)))),
             int(k.process_event(eh.OpSumRows(tv(x, lay), tm(outs["sum_rows"], row_out)))),
             int(k.process_event(eh.OpArgmaxRows(tv(x, lay), tm(outs["argmax_rows"], i32_lay))))]
        return r

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out["captured"] = step()
        out["reserve_under_capture"] = int(eh.stream_reserve(64 << 20, 1 << 20, sid))
    for o in outs.values():
        o.fill_(-7)
    graph.replay()
    s.synchronize()
    got = {n: o.clone() for n, o in outs.items()}
    for o in outs.values():
        o.fill_(-9)
    with torch.cuda.stream(s):
        out["eager"] = step()
    s.synchronize()
    out["replay_matches"] = {n: bool(torch.equal(got[n].view(torch.int32), outs[n].view(torch.int32))) for n in outs}
    graph.replay()  # again, after the eager calls on the same stream and scratch
    s.synchronize()
    out["replay2_matches"] = {n: bool(torch.equal(o.view(torch.int32), got[n].view(torch.int32))) for n, o in outs.items()}
    st, w2, c2 = eh.stream_workspace(sid)
    out["workspace_end"] = [int(st), w2, c2]
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
