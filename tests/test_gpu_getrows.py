"""GPU parity of the row gather (emel_op_get_rows*) with the oracle's
restatement of get_rows.rs, through the C ABI.  Bit-exact for every source
format; rejections (views, shapes, indices) match the oracle's status and
leave dst untouched."""
import numpy as np
import pytest

import emel_hip as eh
import oracle as orc
from helpers import Pair, assert_bits_equal, rng

pytestmark = pytest.mark.gpu

F32, F16, Q4_0, Q8_0, Q4_K, BF16 = 0, 1, 2, 8, 12, 30
EVENTS = {orc.GR_F32: eh.OpGetRows, orc.GR_F32_BYTES: eh.OpGetRowsF32Bytes, orc.GR_F16: eh.OpGetRowsF16,
          orc.GR_BF16: eh.OpGetRowsBf16, orc.GR_Q4_0: eh.OpGetRowsQ4_0, orc.GR_Q8_0: eh.OpGetRowsQ8_0,
          orc.GR_Q4_K: eh.OpGetRowsQ4K}
PACK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144)}


def dense(ne, elem=4):
    nb = [elem]
    for d in range(1, 4):
        nb.append(nb[-1] * ne[d - 1])
    return nb


def packed_nb(code, ne):
    bv, bb = PACK[code]
    row = ne[0] // bv * bb
    return [1, row, row * ne[1], row * ne[1] * ne[2]]


class Gather:
    def __init__(self, gpu):
        import torch

        self.torch = torch
        self.gpu = gpu
        self.kernel = eh.Kernel()

    def __call__(self, kind, src, sne, snb, sdtype, idx, ine, inb=None, dne=None, fill=9.0, src_bytes=None,
                 compare=True, offset=0):
        torch = self.torch
        print(f"get_rows kind={kind} src ne={sne} nb={snb} idx ne={ine} nb={inb}", flush=True)
        dne = dne if dne is not None else [sne[0], ine[0], ine[1], ine[2]]
        count = int(np.prod(dne))
        idx = np.ascontiguousarray(idx, np.int32)
        host_out = np.full(max(count, 1), fill, np.float32)
        sbytes = src.nbytes if src_bytes is None else src_bytes
        want = orc.get_rows(kind, orc.view(src, sne, snb, sdtype, sbytes), orc.index_view(idx, ine, inb),
                            orc.view(host_out, dne, dense(dne), F32, 4 * count))
        # offset: the table starts that many bytes into its allocation (misaligned bases)
        raw = np.zeros(src.nbytes + 16, np.uint8)
        raw[offset:offset + src.nbytes] = src.view(np.uint8)
        dsrc = torch.from_numpy(raw).to(self.gpu)[offset:]
        didx = torch.from_numpy(idx.copy() if idx.size else np.zeros(1, np.int32)).to(self.gpu)
        dout = torch.full((max(count, 1),), fill, dtype=torch.float32, device=self.gpu)
        ev = EVENTS[kind](eh.TensorView(dsrc, eh.Layout(sdtype, sne, snb), sbytes),
                          eh.IndexView(didx, ine, inb, length=idx.size),
                          eh.TensorViewMut(dout, eh.Layout(F32, dne, dense(dne)), 4 * count))
        got = self.kernel.process_event(ev)
        result = dout.cpu().numpy()[:count]
        if compare:
            assert int(got) == want, (kind, want, got, eh.last_error())
            assert_bits_equal(result, host_out[:count], f"get_rows kind {kind}")
            # the same request with host-resident indices (checked in place, passed by value or uploaded)
            dout.fill_(fill)
            hidx = idx.copy() if idx.size else np.zeros(1, np.int32)
            ev = EVENTS[kind](eh.TensorView(dsrc, eh.Layout(sdtype, sne, snb), sbytes),
                              eh.IndexView(hidx, ine, inb, length=idx.size),
                              eh.TensorViewMut(dout, eh.Layout(F32, dne, dense(dne)), 4 * count))
            got_h = self.kernel.process_event(ev)
            assert int(got_h) == want, (kind, "host indices", want, got_h, eh.last_error())
            assert_bits_equal(dout.cpu().numpy()[:count], host_out[:count], f"get_rows kind {kind}, host indices")
        return want, got, result


@pytest.fixture(scope="module")
def gather(gpu):
    return Gather(gpu)


def f32_table(seed, ne):
    x = rng(seed).standard_normal(int(np.prod(ne))).astype(np.float32)
    x[:4] = [np.nan, -0.0, np.inf, 1e-40]
    return x


@pytest.mark.parametrize("cols", [1, 3, 64, 4096, 4097])
def test_f32_dense(gather, cols):
    sne = [cols, 300, 2, 1]
    ine = [50, 2, 1]
    idx = rng(cols).integers(0, 300, 100).astype(np.int32)
    gather(orc.GR_F32, f32_table(cols, sne), sne, dense(sne), F32, idx, ine)


def test_f32_layouts(gather):
    g = rng(7)
    # strided outer dims (rows 20 floats apart, batches apart), implicit nb, non-unit element stride (memcpy)
    sne = [16, 30, 3, 2]
    buf = g.standard_normal(20 * 30 * 3 * 2 + 64).astype(np.float32)
    idx = g.integers(0, 30, 7 * 3 * 2).astype(np.int32)
    gather(orc.GR_F32, buf, sne, [4, 80, 80 * 30, 80 * 90], F32, idx, [7, 3, 2])
    gather(orc.GR_F32, buf, [16, 30, 3, 2], [0, 1, 1, 1], F32, idx, [7, 3, 2])
    gather(orc.GR_F32, buf, [8, 30, 1, 1], [8, 80, 80 * 30, 80 * 30], F32, idx[:7], [7, 1, 1])
    # singleton zero outer strides
    gather(orc.GR_F32, buf[:16].copy(), [16, 1, 1, 1], [4, 0, 0, 0], F32, [0, 0, 0], [3, 1, 1])


def test_f32_strided_and_implicit_indices(gather):
    sne = [33, 10, 2, 1]
    src = f32_table(8, sne)
    raw = rng(9).integers(0, 10, 64).astype(np.int32)
    gather(orc.GR_F32, src, sne, dense(sne), F32, raw, [4, 2, 1], [12, 64, 128])
    gather(orc.GR_F32, src, sne, dense(sne), F32, raw[:8], [4, 2, 1], [0, 2**64 - 1, 3])


def test_f32_bytes_unaligned_rows(gather):
    g = rng(10)
    cols, rows = 5, 12
    row_stride = 4 * cols + 3  # rows start at odd byte offsets
    raw = g.integers(0, 256, row_stride * rows + 8, dtype=np.uint8)
    idx = g.integers(0, rows, 9).astype(np.int32)
    gather(orc.GR_F32_BYTES, raw, [cols, rows, 1, 1], [4, row_stride, row_stride * rows, row_stride * rows],
           F32, idx, [9, 1, 1])


@pytest.mark.parametrize("kind,dtype", [(orc.GR_F16, F16), (orc.GR_BF16, BF16)])
def test_half_sources(gather, kind, dtype):
    g = rng(11)
    sne = [96, 50, 2, 2]
    h = g.integers(0, 65536, int(np.prod(sne)), dtype=np.uint32).astype(np.uint16)  # every pattern class, NaNs too
    idx = g.integers(0, 50, 8 * 2 * 2).astype(np.int32)
    gather(kind, h, sne, dense(sne, 2), dtype, idx, [8, 2, 2])
    # every other column (element stride 4 bytes), and the implicit layout
    gather(kind, h, [48, 50, 1, 1], [4, 192, 192 * 50, 192 * 50], dtype, idx[:8], [8, 1, 1])
    gather(kind, h, sne, [0, 0, 0, 0], dtype, idx, [8, 2, 2])


def all_f16_halves():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)


def test_f16_every_pattern(gather):
    gather(orc.GR_F16, all_f16_halves(), [256, 256, 1, 1], dense([256, 256, 1, 1], 2), F16,
           np.arange(256, dtype=np.int32)[::-1].copy(), [256, 1, 1])


def random_packed(seed, code, sne):
    bv, bb = PACK[code]
    nblk = sne[0] // bv * int(np.prod(sne[1:]))
    g = rng(seed)
    raw = g.integers(0, 256, (nblk, bb), dtype=np.uint8)
    scales = g.standard_normal(nblk * 2).astype(np.float16)
    scales[:3] = [np.inf, np.nan, 6e-8]
    raw[:, :2] = np.frombuffer(scales[:nblk].tobytes(), np.uint8).reshape(nblk, 2)
    if code == Q4_K:
        raw[:, 2:4] = np.frombuffer(scales[nblk:].tobytes(), np.uint8).reshape(nblk, 2)
    return raw.reshape(-1).copy()


@pytest.mark.parametrize("kind,code", [(orc.GR_Q4_0, Q4_0), (orc.GR_Q8_0, Q8_0), (orc.GR_Q4_K, Q4_K)])
def test_quantized(gather, kind, code):
    for cols in (PACK[code][0], 4096):
        sne = [cols, 40, 2, 3]
        src = random_packed(cols + code, code, sne)
        idx = rng(code).integers(0, 40, 5 * 2 * 3).astype(np.int32)
        gather(kind, src, sne, packed_nb(code, sne), code, idx, [5, 2, 3])


def test_embedding_lookup_shapes(gather):
    """The model-facing case: 512 token ids into an [4096, 8192] table."""
    sne = [4096, 8192, 1, 1]
    table = rng(12).standard_normal(4096 * 8192).astype(np.float32)
    ids = rng(13).integers(0, 8192, 512).astype(np.int32)
    gather(orc.GR_F32, table, sne, dense(sne), F32, ids, [512, 1, 1])
    q = random_packed(14, Q4_K, [4096, 2048, 1, 1])
    gather(orc.GR_Q4_K, q, [4096, 2048, 1, 1], packed_nb(Q4_K, [4096, 2048, 1, 1]), Q4_K, ids % 2048, [512, 1, 1])


def test_rejections_and_empty_indices(gather):
    sne = [3, 2, 2, 1]
    src = np.array([1, 2, 3, 4, 5, 6, 10, 20, 30, 40, 50, 60], np.float32)
    cases = [
        ([1, 0, 0, 1], [2, 2, 1], None, [3, 4, 1, 1]),   # shape mismatch
        ([1, -1, 0, 1], [2, 2, 1], None, None),          # negative index
        ([1, 2, 0, 1], [2, 2, 1], None, None),           # index past the rows
        ([1, 0, 0], [2, 2, 1], None, None),              # short index storage
        ([0, 1, 0, 1], [2, 2, 1], [2, 8, 8], None),      # odd index stride
    ]
    for idx, ine, inb, dne in cases:
        want, got, out = gather(orc.GR_F32, src, sne, dense(sne), F32, idx, ine, inb, dne=dne, compare=False)
        assert want != orc.OK and int(got) == want, (idx, ine, inb, want, got)
        assert (out == 9.0).all()
    want, got, _ = gather(orc.GR_F32, src, sne, dense(sne), F32, np.zeros(0, np.int32), [0, 2, 1], [0, 0, 0],
                          dne=[3, 0, 2, 1], compare=False)
    assert want == orc.OK and got == eh.Status.OK
    want, got, out = gather(orc.GR_Q4_0, random_packed(1, Q4_0, [32, 2, 1, 1]), [32, 2, 1, 1], [2, 18, 36, 36],
                            Q4_0, [0], [1, 1, 1], compare=False)
    assert want == orc.INVALID_VIEW and got == eh.Status.INVALID_VIEW and (out == 9.0).all()


def test_misaligned_tables_take_the_element_kernels(gather):
    g = rng(15)
    for kind, code in ((orc.GR_Q4_0, Q4_0), (orc.GR_Q8_0, Q8_0), (orc.GR_Q4_K, Q4_K)):
        sne = [PACK[code][0] * 2, 20, 1, 1]
        src = random_packed(30 + code, code, sne)
        for off in (1, 2):
            gather(kind, src, sne, packed_nb(code, sne), code, g.integers(0, 20, 9).astype(np.int32), [9, 1, 1],
                   offset=off)
    sne = [64, 20, 1, 1]
    h = g.integers(0, 65536, 64 * 20, dtype=np.uint32).astype(np.uint16)
    gather(orc.GR_F16, h, sne, dense(sne, 2), F16, g.integers(0, 20, 9).astype(np.int32), [9, 1, 1], offset=2)
    f = g.standard_normal(64 * 20).astype(np.float32)
    gather(orc.GR_F32, f, sne, dense(sne), F32, g.integers(0, 20, 9).astype(np.int32), [9, 1, 1], offset=4)


def test_more_host_indices_than_the_arguments_carry(gather):
    g = rng(16)
    sne = [256, 1000, 1, 1]
    for kind, code, src in ((orc.GR_F32, F32, f32_table(17, sne)),
                            (orc.GR_Q4_K, Q4_K, random_packed(18, Q4_K, sne))):
        nb = dense(sne) if code == F32 else packed_nb(code, sne)
        gather(kind, src, sne, nb, code, g.integers(0, 1000, 700).astype(np.int32), [700, 1, 1])
