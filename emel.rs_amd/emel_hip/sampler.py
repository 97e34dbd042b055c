"""emel-logits' native sampler and candidate validator over the C ABI.

    sampler = Sampler()
    status, result = sampler.sample_temperature_top_k(SampleTemperatureTopK(
        card, temperature, top_k, logits, sorted_indices, top_probabilities,
        top_indices, random_state, selected_token_out, selected_score_out))
    # status == Status.OK -> result == (token, score)

Mirrors crates/emel-logits/src/sampler/sm.rs (Sampler, SampleTemperatureTopK,
SamplePreselected) and crates/emel-logits/src/validator/sm.rs (Validator,
Build).  Device buffers are torch tensors (float32 / int32, contiguous);
`random_state` is a host numpy uint32 array (one state per row), updated in
place as the reference updates its `&mut u32`.  The calls are synchronous,
like the reference's run-to-completion actors: they wait for the device and
apply the result guard (sampler/sm.rs:849-858) to the outputs.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from .abi import CSampleRequest, CSampleRows, Status, load


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


@dataclass
class SampleTemperatureTopK:
    """SampleTemperatureTopK::new(card, temperature, top_k, logits, sorted_indices,
    top_probabilities, top_indices, random_state, selected_token_out,
    selected_score_out) (sampler/sm.rs:148-195).  `lens` overrides the slice
    lengths (logits, sorted_indices, top_probabilities, top_indices)."""

    card: int
    temperature: float
    top_k: int
    logits: object
    sorted_indices: object
    top_probabilities: object
    top_indices: object
    random_state: np.ndarray
    selected_token_out: object
    selected_score_out: object
    status_out: object = None
    lens: tuple | None = None

    def c(self) -> CSampleRequest:
        if self.random_state.dtype != np.uint32 or not self.random_state.flags["C_CONTIGUOUS"]:
            raise TypeError("random_state must be a contiguous numpy uint32 array")
        lens = self.lens or (self.logits.numel(), self.sorted_indices.numel(), self.top_probabilities.numel(),
                             self.top_indices.numel())
        r = CSampleRequest()
        r.card = self.card
        r.temperature = self.temperature
        r.reserved = 0
        r.top_k = self.top_k
        r.logits, r.logits_len = self.logits.data_ptr(), lens[0]
        r.sorted_indices, r.sorted_indices_len = self.sorted_indices.data_ptr(), lens[1]
        r.top_probabilities, r.top_probabilities_len = self.top_probabilities.data_ptr(), lens[2]
        r.top_indices, r.top_indices_len = self.top_indices.data_ptr(), lens[3]
        r.random_state = self.random_state.ctypes.data
        r.selected_token_out = self.selected_token_out.data_ptr()
        r.selected_score_out = self.selected_score_out.data_ptr()
        r.status_out = None if self.status_out is None else self.status_out.data_ptr()
        return r


@dataclass
class SamplePreselected:
    """SamplePreselected::new(vocab_size, selected_token) (sampler/sm.rs:129-146)."""

    vocab_size: int
    selected_token: int


def _result_valid(token: int, score: float, card: int) -> bool:
    # guard_temperature_result_valid (sampler/sm.rs:849-858)
    return 0 <= token < card and np.isfinite(score)


class Sampler:
    """The logits sampler actor (sampler/sm.rs:303-393) on one HIP stream."""

    def __init__(self, stream: int | None = None):
        self._lib = load()
        self.stream = stream

    def _sync(self) -> Status:
        return Status(self._lib.emel_stream_synchronize(self.stream))

    def sample_temperature_top_k(self, req: SampleTemperatureTopK):
        """-> (Status.OK, (token, score)) or (error status, None)."""
        c = req.c()
        st = Status(self._lib.emel_sample_temperature_top_k(ctypes.byref(c), self.stream))
        if st != Status.OK:
            return st, None
        sync = self._sync()
        if sync != Status.OK:
            return sync, None
        token = int(req.selected_token_out.reshape(-1)[0].item())
        score = float(req.selected_score_out.reshape(-1)[0].item())
        if not _result_valid(token, score, req.card):
            return Status.INVALID_REQUEST, None
        return Status.OK, (token, score)

    def sample_temperature_top_k_rows(self, req: SampleTemperatureTopK, rows: int, logits_stride: int,
                                      sorted_stride: int, top_stride: int):
        """`rows` requests at once (emel_sample_temperature_top_k_rows).
        -> (Status.OK, [(token, score) | Status.INVALID_REQUEST per row]) or (error, None)."""
        c = req.c()
        cr = CSampleRows(rows, logits_stride, sorted_stride, top_stride)
        st = Status(self._lib.emel_sample_temperature_top_k_rows(ctypes.byref(c), ctypes.byref(cr), self.stream))
        if st != Status.OK:
            return st, None
        sync = self._sync()
        if sync != Status.OK:
            return sync, None
        toks = req.selected_token_out.reshape(-1)[:rows].cpu().numpy()
        scores = req.selected_score_out.reshape(-1)[:rows].cpu().numpy()
        out = []
        for t, s in zip(toks, scores):
            out.append((int(t), float(s)) if _result_valid(int(t), float(s), req.card) else Status.INVALID_REQUEST)
        return Status.OK, out

    def sample_preselected(self, req: SamplePreselected):
        """-> (Status.OK, token) or (Status.INVALID_REQUEST, None) (sampler/sm.rs:366-378)."""
        tok = ctypes.c_int32(0)
        st = Status(self._lib.emel_sample_preselected(req.vocab_size, req.selected_token, ctypes.byref(tok)))
        return (st, int(tok.value)) if st == Status.OK else (st, None)


@dataclass
class Build:
    """Build::new(logits, vocab_size, candidate_ids, candidate_scores,
    candidate_capacity, candidate_count_out, error_out) (validator/sm.rs:33-66).
    The count and error outputs are the fields below, written by the call."""

    logits: object
    vocab_size: int
    candidate_ids: object
    candidate_scores: object
    candidate_capacity: int
    candidate_count_out: int = -1
    error_out: int = -1  # ValidatorError discriminant: 0 None, 1 InvalidRequest
    lens: tuple | None = field(default=None)


class Validator:
    """The logits validator actor (validator/sm.rs:242-262)."""

    def __init__(self, stream: int | None = None):
        self._lib = load()
        self.stream = stream

    def process_event(self, req: Build):
        """-> (Status.OK, candidate_count) or (error status, None)."""
        lens = req.lens or (req.logits.numel(), req.candidate_ids.numel(), req.candidate_scores.numel())
        count = ctypes.c_int32(req.candidate_count_out)
        err = ctypes.c_int32(req.error_out)
        st = Status(self._lib.emel_logits_validator_build(
            _ptr(req.logits), lens[0], req.vocab_size, _ptr(req.candidate_ids), lens[1], _ptr(req.candidate_scores),
            lens[2], req.candidate_capacity, ctypes.byref(count), ctypes.byref(err), self.stream))
        req.candidate_count_out = int(count.value)
        req.error_out = int(err.value)
        if st != Status.OK:
            return st, None
        sync = Status(self._lib.emel_stream_synchronize(self.stream))
        if sync != Status.OK:
            return sync, None
        return Status.OK, req.candidate_count_out
