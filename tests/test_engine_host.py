"""Host logic of klsample.engine on the CPU: device-history bookkeeping (with the
library's append emulated), batching of per-request logits, the SSE wire format."""
import json

import numpy as np
import pytest
import torch

from klsample import engine as eng


def _append(h, slots, ranges, tokens):
    """What the library does with history_append: row b's token at arena[end_b]."""
    for b, t in enumerate(tokens):
        h.arena[int(ranges[2 * b + 1])] = t
    h.advance(slots)


def test_device_history_keeps_prompt_plus_generated():
    rng = np.random.default_rng(0)
    V = 1000
    h = eng.DeviceHistory('cpu', V, capacity=1024, reserve=2)
    want = {}
    for r in range(70):                     # past the 64 initial slots
        ids = rng.integers(-V, V, int(rng.integers(0, 40))).tolist()
        h.register(r, ids)
        want[r] = [i % V for i in ids]
    live = list(range(70))
    for step in range(40):
        rids = live[step % 3::2] or live
        slots = h.slots(rids)
        ranges = h.prepare(slots)
        for b, r in enumerate(rids):         # ranges are disjoint and have a free slot after them
            s = h.slot[r]
            assert ranges[2 * b] == h.start[s] and ranges[2 * b + 1] - ranges[2 * b] == len(want[r])
            assert ranges[2 * b + 1] < h.start[s] + h.cap[s]
        toks = rng.integers(0, V, len(rids)).tolist()
        _append(h, slots, ranges, toks)
        for r, t in zip(rids, toks):
            want[r].append(t)
        if step % 7 == 6:                    # release some; new requests reuse the segments
            for r in live[:3]:
                h.release(r)
                del want[r]
            live = live[3:]
            nr = 1000 + step
            h.register(nr, [1, 2, 3])
            want[nr] = [1, 2, 3]
            live.append(nr)
    for r in live:
        assert h.ids(r).tolist() == want[r]
    # segments of live requests never overlap
    segs = sorted((int(h.start[h.slot[r]]), int(h.cap[h.slot[r]])) for r in live)
    assert all(a + c <= b for (a, c), (b, _) in zip(segs, segs[1:]))


def test_device_history_rejects_ids_the_reference_would_not_index():
    h = eng.DeviceHistory('cpu', 10)
    with pytest.raises(IndexError):
        h.register('a', [3, 10])
    h.register('b', [-1, 0])
    assert h.ids('b').tolist() == [9, 0]
    with pytest.raises(KeyError):
        h.register('b', [])


def test_per_request_rows_of_one_tensor_are_used_in_place():
    x = torch.randn(5, 7)
    d = {f'r{i}': x[i] for i in range(5)}
    b = eng.as_batch(d, ['r1', 'r2', 'r3'])
    assert b.data_ptr() == x[1].data_ptr() and torch.equal(b, x[1:4])
    b = eng.as_batch(d, ['r3', 'r1'])          # not evenly spaced upward: stacked
    assert torch.equal(b, x[[3, 1]])
    assert torch.equal(eng.as_batch({'a': x[2]}, ['a']), x[2:3])
    assert eng.as_batch(x, None) is x


def test_sse_chunks_follow_the_reference_wire_format():
    """serving/api.py:62-68: a token chunk and a finish chunk, text and chat."""
    ev = eng.TokenEvent('cmpl-9', 17, -0.25, ((17, -0.25), (3, -1.5)))
    line = eng.sse_chunk(ev, text='ab')
    assert line == ('data: {"id": "cmpl-9", "object": "text_completion", "choices": [{"index": 0, '
                    '"finish_reason": null, "logprobs": {"token_logprob": -0.25, "top_logprobs": '
                    '[[17, -0.25], [3, -1.5]]}, "text": "ab"}]}\n\n')
    chat = json.loads(eng.sse_chunk(ev, text='ab', chat=True)[6:])
    assert chat['object'] == 'chat.completion.chunk' and chat['choices'][0]['delta'] == {'content': 'ab'}
    assert 'text' not in chat['choices'][0]
    done = eng.sse_chunk(eng.TokenEvent('cmpl-9', finished=True, finish_reason='length'))
    assert done == ('data: {"id": "cmpl-9", "object": "text_completion", "choices": [{"index": 0, '
                    '"delta": null, "text": "", "finish_reason": "length"}]}\n\n')
    done = json.loads(eng.sse_chunk(eng.TokenEvent('x', finished=True, finish_reason='stop'), chat=True)[6:])
    assert done['choices'][0] == {'index': 0, 'delta': {}, 'text': None, 'finish_reason': 'stop'}
    assert eng.SSE_DONE == 'data: [DONE]\n\n'
