"""klsample_run_noalloc against klsample_run, through the C ABI (MI355X only).

The no-allocation entry point runs the same kernels in a static device array instead
of a caller workspace; its outputs must equal klsample_run's bit for bit, on two calls
in a row of which the second is smaller (the scratch keeps the first call's contents)."""
import ctypes
import sys

import numpy as np
import pytest
import torch

from klsample import SamplingParams, _lib, workloads
from klsample.runner import pack_rows

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _call(lib, fn, logits, params, hist, uniforms, n, workspace):
    """One call of `fn` (klsample_run or klsample_run_noalloc) on device tensors; returns
    host copies of every output."""
    B, V = logits.shape
    rows, offsets, ids, max_top_k = pack_rows(params, hist, uniforms, V)
    d_rows = torch.from_numpy(rows.view(np.uint8).copy()).to(DEV)
    d_off = torch.from_numpy(offsets).to(DEV)
    d_ids = torch.from_numpy(ids if ids.size else np.zeros(1, np.int32)).to(DEV)
    tok = torch.full((B,), -7, dtype=torch.int64, device=DEV)
    lp = torch.full((B,), float('nan'), dtype=torch.float32, device=DEV)
    tid = torch.full((max(B * n, 1),), -7, dtype=torch.int32, device=DEV)
    tlp = torch.full((max(B * n, 1),), float('nan'), dtype=torch.float32, device=DEV)
    info = torch.zeros(B * _lib.ROW_INFO_DTYPE.itemsize, dtype=torch.uint8, device=DEV)
    b = _lib.Batch()
    b.logits = logits.data_ptr()
    b.row_stride = V
    b.dtype = _lib.FLOAT32 if logits.dtype == torch.float32 else _lib.BFLOAT16
    b.batch, b.vocab, b.num_logprobs, b.max_top_k, b.options = B, V, n, max_top_k, 0
    b.params = d_rows.data_ptr()
    b.history_ids = d_ids.data_ptr() if ids.size else None
    b.history_offsets = d_off.data_ptr() if ids.size else None
    b.token_ids, b.logprobs = tok.data_ptr(), lp.data_ptr()
    b.top_ids = tid.data_ptr() if n else None
    b.top_logprobs = tlp.data_ptr() if n else None
    b.probs = None
    b.row_info = info.data_ptr()
    if workspace is None:
        b.workspace, b.workspace_bytes = None, 0
    else:
        b.workspace, b.workspace_bytes = workspace
    stream = torch.cuda.current_stream(DEV).cuda_stream
    _lib.check(lib, fn(ctypes.byref(b), ctypes.c_void_p(stream)))
    torch.cuda.synchronize()
    return (tok.cpu().numpy(), lp.cpu().numpy(), tid.cpu().numpy(), tlp.cpu().numpy(),
            info.cpu().numpy().view(_lib.ROW_INFO_DTYPE))


def _same(a, b):
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8))


def test_noalloc_matches_run_on_two_calls_the_second_smaller():
    lib = _lib.load()
    n = 5
    first = workloads.make('mixed_b64', batch=24, num_logprobs=n)
    rng = np.random.default_rng(41)
    V2 = 20011
    x2 = torch.from_numpy((rng.standard_normal((3, V2)) * 2).astype(np.float32))
    p2 = [SamplingParams(temperature=0.8, top_k=30, top_p=0.9, logprobs=n),
          SamplingParams(repetition_penalty=1.3, logprobs=n),
          SamplingParams(temperature=1.1, top_p=0.7, logprobs=n)]
    h2 = [rng.integers(0, V2, 40).tolist() for _ in range(3)]
    u2 = rng.random(3).astype(np.float32)
    cases = [(first.logits, first.params, first.histories, first.uniforms), (x2, p2, h2, u2)]
    for step, (x, params, hist, u) in enumerate(cases):
        say(f'no-alloc call {step}: B={x.shape[0]} V={x.shape[1]} dtype={x.dtype}')
        d = x.to(DEV)
        dt = _lib.FLOAT32 if d.dtype == torch.float32 else _lib.BFLOAT16
        need = _lib.workspace_size(d.shape[0], d.shape[1], dt, max((p.top_k for p in params), default=0), n)
        assert need <= _lib.NOALLOC_SCRATCH_BYTES
        ws = torch.empty(need + 256, dtype=torch.uint8, device=DEV)
        wptr = ws.data_ptr() + (-ws.data_ptr()) % 256
        want = _call(lib, lib.klsample_run, d, params, hist, u, n, (wptr, need))
        got = _call(lib, lib.klsample_run_noalloc, d, params, hist, u, n, None)
        _same(got, want)
        # and again: the scratch now holds this call's own contents
        _same(_call(lib, lib.klsample_run_noalloc, d, params, hist, u, n, None), want)
        say(f'  tokens equal: {want[0][:6].tolist()}...')
