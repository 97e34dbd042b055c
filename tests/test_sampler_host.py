"""CPU: the host side of the sampler / validator C ABI -- the reference's
request guards (emel-logits sampler/sm.rs:729-747, :685-695,
validator/sm.rs:177-190) and the C ABI's own argument checks run before
anything touches a device, and a rejected call writes nothing (the host
random_state included).  No kernel is launched."""
import ctypes

import numpy as np
import pytest
import torch

import emel_hip as eh
from emel_hip.abi import CSampleRequest, CSampleRows

M = 2147483647


def request(card=8, top_k=3, temperature=1.0, states=(7,), rows=1, **over):
    t = dict(
        logits=torch.zeros(card * rows, dtype=torch.float32),
        sorted_indices=torch.zeros(card * rows, dtype=torch.int32),
        top_probabilities=torch.zeros(top_k * rows, dtype=torch.float32),
        top_indices=torch.zeros(top_k * rows, dtype=torch.int32),
        selected_token_out=torch.zeros(rows, dtype=torch.int32),
        selected_score_out=torch.zeros(rows, dtype=torch.float32),
    )
    t.update(over)
    rs = np.array(states, np.uint32)
    req = eh.SampleTemperatureTopK(card, temperature, top_k, t["logits"], t["sorted_indices"],
                                   t["top_probabilities"], t["top_indices"], rs, t["selected_token_out"],
                                   t["selected_score_out"])
    return req, rs


def call(req, rows=None):
    lib = eh.load()
    c = req.c()
    if rows is None:
        return eh.Status(lib.emel_sample_temperature_top_k(ctypes.byref(c), None))
    cr = CSampleRows(*rows)
    return eh.Status(lib.emel_sample_temperature_top_k_rows(ctypes.byref(c), ctypes.byref(cr), None))


@pytest.mark.parametrize("kw", [dict(card=0), dict(top_k=0), dict(top_k=9), dict(temperature=0.0),
                                dict(temperature=-2.0), dict(temperature=float("inf")),
                                dict(temperature=float("nan")), dict(states=(0,)), dict(states=(M,))])
def test_request_guard(kw):
    args = dict(card=8, top_k=3)
    args.update(kw)
    req, rs = request(**args) if args["card"] else request(card=8, top_k=3)
    if args["card"] == 0:
        req.card = 0
    before = rs.copy()
    assert call(req) == eh.Status.INVALID_REQUEST
    assert np.array_equal(rs, before)


@pytest.mark.parametrize("which,short", [(0, 7), (1, 7), (2, 2), (3, 2)])
def test_slice_lengths_are_guarded(which, short):
    req, rs = request()
    lens = [8, 8, 3, 3]
    lens[which] = short
    req.lens = tuple(lens)
    assert call(req) == eh.Status.INVALID_REQUEST and rs[0] == 7


def test_batch_rejects_when_any_row_fails():
    req, rs = request(rows=3, states=(7, 2 * M, 9))
    assert call(req, (3, 8, 8, 3)) == eh.Status.INVALID_REQUEST
    assert rs.tolist() == [7, 2 * M, 9]
    req, rs = request(rows=3, states=(7, 8, 9))
    assert call(req, (3, 7, 8, 3)) == eh.Status.INVALID_REQUEST  # rows of logits would overlap
    assert call(req, (0, 8, 8, 3)) == eh.Status.INVALID_ARGUMENT


def test_argument_checks():
    req, rs = request()
    c = req.c()
    c.selected_token_out = None
    assert eh.Status(eh.load().emel_sample_temperature_top_k(ctypes.byref(c), None)) == eh.Status.INVALID_ARGUMENT
    c = req.c()
    c.reserved = 1
    assert eh.Status(eh.load().emel_sample_temperature_top_k(ctypes.byref(c), None)) == eh.Status.INVALID_ARGUMENT
    shared = torch.zeros(16, dtype=torch.int32)
    req, rs = request(sorted_indices=shared[:8], top_indices=shared[6:9])
    req.lens = (8, 8, 3, 3)
    assert call(req) == eh.Status.INVALID_ARGUMENT
    raw = torch.zeros(64, dtype=torch.uint8)
    req, rs = request()
    c = req.c()
    c.logits = raw.data_ptr() + 2
    assert eh.Status(eh.load().emel_sample_temperature_top_k(ctypes.byref(c), None)) == eh.Status.INVALID_ARGUMENT
    assert rs[0] == 7


def test_accepted_request_without_gpu_is_kernel_unavailable():
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    req, rs = request()
    assert call(req) == eh.Status.KERNEL_UNAVAILABLE
    assert rs[0] == 7  # nothing was drawn


def test_sample_preselected():
    s = eh.Sampler()
    assert s.sample_preselected(eh.SamplePreselected(3, 2)) == (eh.Status.OK, 2)
    for vocab, tok in [(3, 3), (0, 0), (3, -1)]:
        assert s.sample_preselected(eh.SamplePreselected(vocab, tok)) == (eh.Status.INVALID_REQUEST, None)


@pytest.mark.parametrize("vocab,capacity", [(0, 2), (2, 1), (-1, 2), (3, 3)])
def test_validator_guard_resets_outputs(vocab, capacity):
    # tests/validator.rs: build_rejects_invalid_sizes_and_resets_outputs
    b = eh.Build(torch.tensor([1.0, 2.0]), vocab, torch.full((2,), 7, dtype=torch.int32),
                 torch.full((2,), 8.0), capacity, candidate_count_out=9, error_out=2)
    st, _ = eh.Validator().process_event(b)
    assert st == eh.Status.INVALID_REQUEST
    assert b.candidate_count_out == 0 and b.error_out == 1
