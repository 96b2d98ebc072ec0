"""Seeded synthetic workloads of the sampling path.

Each workload is a ``[B, V]`` logits matrix on the host, one ``SamplingParams`` per
row, per-row token histories and per-row uniforms.  Generation uses numpy's PCG64
seeded with ``20261201 + n`` for workload family ``n``; bf16 logits are the
round-to-nearest-even bf16 values of the fp32 draws.

=====================================  ======  =======  ======  ==========================
name                                   B       V        dtype   rows
=====================================  ======  =======  ======  ==========================
cpu_reference_b8                       8       151936   fp32    0-3 greedy; 4-7 T=.8 k=50 p=.9
latency_b1                             1       151936   bf16    T=.7 p=.95 (heavy head)
latency_b1_greedy                      1       151936   bf16    greedy (same logits)
mixed_b64                              64      151936   bf16    mixed T/k/p, all penalties, H=512
throughput_b256_v128256                256     128256   fp32    T=1 k=40 p=.9, penalties, H=2048
throughput_b256_v151936                256     151936   fp32    as above at V=151936
tie_stress_b1024                       1024    151936   fp32    bf16-grid ties; half greedy, H=4096
=====================================  ======  =======  ======  ==========================
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np
import torch

from .sampling import SamplingParams

QWEN3_VOCAB = 151936
LLAMA32_VOCAB = 128256

NAMES = (
    'cpu_reference_b8',
    'latency_b1',
    'latency_b1_greedy',
    'mixed_b64',
    'throughput_b256_v128256',
    'throughput_b256_v151936',
    'tie_stress_b1024',
)


@dataclass
class Workload:
    name: str
    logits: torch.Tensor            # host [B, V], float32 or bfloat16
    params: list                    # SamplingParams per row
    histories: list                 # np.int32 arrays per row
    uniforms: np.ndarray            # float32 [B]

    @property
    def batch(self) -> int:
        return self.logits.shape[0]

    @property
    def vocab(self) -> int:
        return self.logits.shape[1]

    @property
    def history_tokens(self) -> int:
        return int(sum(len(h) for h, p in zip(self.histories, self.params) if _penalised(p)))

    def algorithmic_bytes(self) -> int:
        """Bytes one call must move: every logit once, every penalising history id once,
        plus per-row parameters (32 B), uniform-free outputs (token 8 B, logprob 4 B) and
        CSR offsets (4 B)."""
        elem = self.logits.element_size()
        return self.batch * self.vocab * elem + 4 * self.history_tokens + self.batch * (32 + 8 + 4 + 4)


def digest(w: Workload) -> str:
    """SHA-256 of everything a workload feeds the sampler: the logits' bytes, the
    uniforms, every history (length then ids) and every row's parameters.  The committed
    digests detect a change of the generator (numpy's PCG64 streams, the bf16 rounding)
    between machines."""
    h = hashlib.sha256()
    h.update(str((tuple(w.logits.shape), str(w.logits.dtype))).encode())
    h.update(w.logits.contiguous().view(torch.uint8).numpy().tobytes())
    h.update(np.ascontiguousarray(w.uniforms, dtype=np.float32).tobytes())
    for hist in w.histories:
        ids = np.ascontiguousarray(hist, dtype=np.int32)
        h.update(np.int64(ids.size).tobytes())
        h.update(ids.tobytes())
    for p in w.params:
        h.update(repr((p.temperature, p.top_k, p.top_p, p.repetition_penalty, sorted(p.stop_token_ids), p.seed,
                       p.logprobs, p.presence_penalty, p.frequency_penalty)).encode())
    return h.hexdigest()


def _penalised(p) -> bool:
    return p.repetition_penalty != 1 or p.presence_penalty != 0 or p.frequency_penalty != 0


def _zipf_ids(rng: np.random.Generator, vocab: int, s: float, count: int, rows: int) -> list:
    """Truncated Zipf(s) over ranks 1..vocab, mapped to token ids through a seeded permutation."""
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    perm = rng.permutation(vocab).astype(np.int32)
    out = []
    for _ in range(rows):
        r = np.searchsorted(cdf, rng.random(count), side='right')
        out.append(perm[np.minimum(r, vocab - 1)])
    return out


def _bf16(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(x).to(torch.bfloat16)


def make(name: str, *, batch: int | None = None, num_logprobs: int = 0) -> Workload:
    """Build workload ``name``; ``batch`` truncates it to its first rows (parity tests at
    reduced size use the same rows as the full workload)."""
    if name == 'cpu_reference_b8':
        rng = np.random.Generator(np.random.PCG64(20261201 + 1))
        B, V = 8, QWEN3_VOCAB
        logits = torch.from_numpy((rng.standard_normal((B, V)) * 2.0).astype(np.float32))
        params = [SamplingParams(logprobs=num_logprobs) for _ in range(4)] + [
            SamplingParams(temperature=0.8, top_k=50, top_p=0.9, logprobs=num_logprobs) for _ in range(4)]
        hist = [np.zeros(0, np.int32)] * B
        u = rng.random(B).astype(np.float32)
    elif name in ('latency_b1', 'latency_b1_greedy'):
        rng = np.random.Generator(np.random.PCG64(20261201 + 2))
        V = QWEN3_VOCAB
        x = (rng.standard_normal(V) * 3.0).astype(np.float32)
        heavy = rng.choice(V, size=round(V * 0.001), replace=False)
        x[heavy] += 8.0
        logits = _bf16(x[None, :])
        if name == 'latency_b1':
            params = [SamplingParams(temperature=0.7, top_p=0.95, logprobs=num_logprobs)]
        else:
            params = [SamplingParams(logprobs=num_logprobs)]
        hist = [np.zeros(0, np.int32)]
        u = rng.random(1).astype(np.float32)
    elif name == 'mixed_b64':
        rng = np.random.Generator(np.random.PCG64(20261201 + 3))
        B, V = 64, QWEN3_VOCAB
        logits = _bf16((rng.standard_normal((B, V)) * 2.5).astype(np.float32))
        temps = rng.uniform(0.5, 1.5, B)
        ks = rng.choice([0, 20, 50, 1000], size=B)
        ps = rng.uniform(0.8, 1.0, B)
        params = [SamplingParams(temperature=float(temps[b]), top_k=int(ks[b]), top_p=float(ps[b]),
                                 repetition_penalty=1.1, logprobs=num_logprobs,
                                 presence_penalty=0.5, frequency_penalty=0.3) for b in range(B)]
        hist = [rng.integers(0, V, 512).astype(np.int32) for _ in range(B)]
        u = rng.random(B).astype(np.float32)
    elif name in ('throughput_b256_v128256', 'throughput_b256_v151936'):
        rng = np.random.Generator(np.random.PCG64(20261201 + 4))
        B = 256
        V = LLAMA32_VOCAB if name.endswith('128256') else QWEN3_VOCAB
        logits = torch.from_numpy((rng.standard_normal((B, V)) * 3.0).astype(np.float32))
        params = [SamplingParams(temperature=1.0, top_k=40, top_p=0.9, repetition_penalty=1.1,
                                 logprobs=num_logprobs, presence_penalty=0.5, frequency_penalty=0.3)
                  for _ in range(B)]
        hist = _zipf_ids(rng, V, 1.1, 2048, B)
        u = rng.random(B).astype(np.float32)
    elif name == 'tie_stress_b1024':
        rng = np.random.Generator(np.random.PCG64(20261201 + 5))
        B, V = 1024, QWEN3_VOCAB
        logits = _bf16((rng.standard_normal((B, V)) * 2.0).astype(np.float32)).float()
        params = [SamplingParams(repetition_penalty=1.2, logprobs=num_logprobs) if b % 2 == 0 else
                  SamplingParams(temperature=0.9, top_k=100, top_p=0.95, repetition_penalty=1.2,
                                 logprobs=num_logprobs) for b in range(B)]
        hist = _zipf_ids(rng, V, 1.1, 4096, B)
        u = rng.random(B).astype(np.float32)
    else:
        raise KeyError(f'unknown workload {name!r}; known: {", ".join(NAMES)}')
    w = Workload(name, logits, params, list(hist), u)
    if batch is not None and batch < w.batch:
        w = Workload(name, w.logits[:batch].contiguous(), w.params[:batch], w.histories[:batch], w.uniforms[:batch])
    return w
