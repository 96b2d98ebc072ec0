"""Throughput and latency of the fused token-sampling path on one MI355X.

A *step* is one ``klsample_run`` over one batch of synthetic input that is already
resident in HBM: the B=256, V=151936 fp32 batch (temperature 1.0, top_k 40,
top_p 0.9, repetition 1.1, presence 0.5, frequency 0.3, 2048-token Zipf(1.1)
histories per row).  Successive steps read identical copies of that batch from
different HBM buffers (together larger than twice the 256 MiB last-level cache), so
every step streams its logits from HBM.

Printed on one JSON line:

* ``value``: sampled rows/s of the whole call (wall clock between synchronisations);
* ``roofline``: algorithmic bytes of one call / the streaming-pass kernel's average
  duration (HIP events recorded on the launch stream around that kernel, through
  ``klsample_set_phase_events``), against the 8 TB/s HBM peak; ``traffic`` is the
  kernel's measured HBM bytes per launch from the committed rocprofv3 counter summary
  (``profiles/traffic_scan_kernel_f32_b256_v151936.txt``), or null when absent;
  ``whole_call_frac`` is the same bytes over the whole call's device time (both kernels
  and the gaps between calls);
* ``b1_latency_us``: device time per call at B=1, V=151936 bf16 (sampled and greedy:
  the mean of 1000 back-to-back calls, and the median and largest of 100 groups of 10),
  and the host wall time of one ``Sampler.sample`` call;
* ``cpu_baseline``: the CPU restatement of ``serving/sampling.py:44-63`` in its
  faithful mode (``torch.multinomial`` draw), one call per row as
  ``serving/engine.py:92-96`` makes them, on the host's cores.

Other modes (used to produce the text summaries under ``profiles/``):

* ``--profile-run [--workload NAME]``: only the steps of one workload (the headline by
  default) and a 1 GiB copy that calibrates HBM byte counters; meant to run under
  ``rocprofv3 --pmc``;
* ``--lmhead``: the fused LM head + sampling call against a bf16 matmul followed by the
  sampling call;
* ``--summarize-stats DIR`` / ``--summarize-pmc FETCH_DIR WRITE_DIR``: turn the CSV
  output of rocprofv3 into those summaries;
* ``--summarize-parity JSONL``: the per-case parity counts the GPU tests log.
"""
from __future__ import annotations

import argparse
import csv
import ctypes
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / 'gpu-kernel-lab_amd', ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = 'sampled rows/s + HBM GB/s at B=256,V=151936; B=1 sample latency µs'
HEADLINE = 'throughput_b256_v151936'
PEAK_HBM_GBS = 8000.0
MALL_BYTES = 256 << 20
COPY_CALIBRATION_BYTES = 1 << 30
TRAFFIC_SUMMARY = ROOT / 'profiles' / 'traffic_scan_kernel_f32_b256_v151936.txt'


# ---- HIP events through the runtime torch already loaded -------------------------------------

class HipEvents:
    """hipEvent_t handles via ctypes (same libamdhip64 as torch: dlopen reuses the soname).

    Events are created with hipEventDisableSystemFence: recording them then costs no
    system-scope cache writeback/invalidate, which would otherwise lengthen the interval
    they bracket and slow the kernel after them.  Results are read only after a full
    device synchronisation."""

    DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self):
        self.hip = ctypes.CDLL('libamdhip64.so.7')
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def _ok(self, status, what):
        if status != 0:
            raise RuntimeError(f'{what} failed with hipError {status}')

    def create(self, n):
        out = []
        for _ in range(n):
            h = ctypes.c_void_p()
            self._ok(self.hip.hipEventCreateWithFlags(ctypes.byref(h), self.DISABLE_SYSTEM_FENCE),
                     'hipEventCreateWithFlags')
            out.append(h.value)
        return out

    def record(self, ev, stream):
        self._ok(self.hip.hipEventRecord(ctypes.c_void_p(ev), ctypes.c_void_p(stream)), 'hipEventRecord')

    def elapsed_ms(self, a, b):
        self._ok(self.hip.hipEventSynchronize(ctypes.c_void_p(b)), 'hipEventSynchronize')
        ms = ctypes.c_float()
        self._ok(self.hip.hipEventElapsedTime(ctypes.byref(ms), ctypes.c_void_p(a), ctypes.c_void_p(b)),
                 'hipEventElapsedTime')
        return float(ms.value)

    def destroy(self, evs):
        for e in evs:
            self.hip.hipEventDestroy(ctypes.c_void_p(e))


# ---- one workload resident in HBM ----------------------------------------------------------

class Resident:
    """Device copies of a workload's logits (rotated), parameters, history and outputs,
    and the ``klsample_batch`` that launches it."""

    def __init__(self, name, device, num_logprobs=0):
        import numpy as np
        import torch
        from klsample import _lib, workloads
        from klsample.runner import pack_rows

        self.lib = _lib.load()
        self.w = w = workloads.make(name, num_logprobs=num_logprobs)
        B, V = w.batch, w.vocab
        rows, offsets, ids, max_top_k = pack_rows(w.params, w.histories, w.uniforms, V)
        size = w.logits.numel() * w.logits.element_size()
        self.copies = max(1, -(-2 * MALL_BYTES // size) + 1) if size * 4 > MALL_BYTES else 1
        first = w.logits.to(device)
        self.logits = [first] + [first.clone() for _ in range(self.copies - 1)]
        self.d_rows = torch.from_numpy(rows.view(np.uint8).copy()).to(device)
        self.d_off = torch.from_numpy(offsets).to(device)
        self.d_ids = torch.from_numpy(ids if ids.size else np.zeros(1, np.int32)).to(device)
        N = num_logprobs
        self.token = torch.empty(B, dtype=torch.int64, device=device)
        self.logprob = torch.empty(B, dtype=torch.float32, device=device)
        self.top_ids = torch.empty(max(B * N, 1), dtype=torch.int32, device=device)
        self.top_lp = torch.empty(max(B * N, 1), dtype=torch.float32, device=device)
        dt = _lib.FLOAT32 if w.logits.dtype == torch.float32 else _lib.BFLOAT16
        ws = _lib.workspace_size(B, V, dt, max_top_k, N)
        self.ws = torch.empty(ws + 256, dtype=torch.uint8, device=device)
        ws_ptr = self.ws.data_ptr() + (-self.ws.data_ptr()) % 256
        self.stream = torch.cuda.current_stream(device).cuda_stream
        _lib.check(self.lib, self.lib.klsample_workspace_init(ctypes.c_void_p(ws_ptr), ctypes.c_size_t(ws),
                                                              ctypes.c_void_p(self.stream)))
        b = self.batch = _lib.Batch()
        b.row_stride = V
        b.dtype = dt
        b.batch = B
        b.vocab = V
        b.num_logprobs = N
        b.max_top_k = max_top_k
        b.options = 0
        b.params = self.d_rows.data_ptr()
        b.history_ids = self.d_ids.data_ptr() if ids.size else None
        b.history_offsets = self.d_off.data_ptr() if ids.size else None
        b.token_ids = self.token.data_ptr()
        b.logprobs = self.logprob.data_ptr()
        b.top_ids = self.top_ids.data_ptr() if N else None
        b.top_logprobs = self.top_lp.data_ptr() if N else None
        b.workspace = ws_ptr
        b.workspace_bytes = ws
        self._ref = ctypes.byref(b)
        self._stream = ctypes.c_void_p(self.stream)
        self._ptrs = [t.data_ptr() for t in self.logits]
        self.alg_bytes = w.algorithmic_bytes()

    def launch(self, i):
        self.batch.logits = self._ptrs[i % self.copies]
        st = self.lib.klsample_run(self._ref, self._stream)
        if st != 0:
            from klsample import _lib
            _lib.check(self.lib, st)


def timed_steps(res, steps, warmup):
    """Wall-clock and event time of ``steps`` back-to-back calls after ``warmup``."""
    import torch
    for i in range(warmup):
        res.launch(i)
    torch.cuda.synchronize()
    hip = HipEvents()
    e0, e1 = hip.create(2)
    t0 = time.perf_counter()
    hip.record(e0, res.stream)
    for i in range(steps):
        res.launch(i)
    hip.record(e1, res.stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dev_ms = hip.elapsed_ms(e0, e1)
    hip.destroy([e0, e1])
    return wall * 1e3 / steps, dev_ms / steps


def per_call_us(res, groups, per_group, warmup):
    """Device time per call (µs) of ``groups`` groups of ``per_group`` back-to-back calls:
    HIP events recorded on the launch stream between the groups (a marker between every
    call would add its own cost to each).  Returns the sorted per-group averages."""
    import torch
    for i in range(warmup):
        res.launch(i)
    hip = HipEvents()
    evs = hip.create(groups + 1)
    torch.cuda.synchronize()
    hip.record(evs[0], res.stream)
    for g in range(groups):
        for i in range(per_group):
            res.launch(g * per_group + i)
        hip.record(evs[g + 1], res.stream)
    torch.cuda.synchronize()
    out = sorted(hip.elapsed_ms(evs[g], evs[g + 1]) * 1e3 / per_group for g in range(groups))
    hip.destroy(evs)
    return out


def phase_times(res, steps):
    """Average duration (ms) of the streaming pass and of the row combine, from HIP events
    the library records around each kernel of each call."""
    import torch
    hip = HipEvents()
    evs = hip.create(3 * steps)
    arr = (ctypes.c_void_p * 3)()
    torch.cuda.synchronize()
    try:
        for i in range(steps):
            arr[0], arr[1], arr[2] = evs[3 * i], evs[3 * i + 1], evs[3 * i + 2]
            res.lib.klsample_set_phase_events(arr, 3)
            res.launch(i)
    finally:
        res.lib.klsample_set_phase_events(None, 0)
    torch.cuda.synchronize()
    scan = sum(hip.elapsed_ms(evs[3 * i], evs[3 * i + 1]) for i in range(steps)) / steps
    comb = sum(hip.elapsed_ms(evs[3 * i + 1], evs[3 * i + 2]) for i in range(steps)) / steps
    hip.destroy(evs)
    return scan, comb


def read_traffic():
    """Measured HBM bytes per launch of the streaming pass (committed counter summary)."""
    if not TRAFFIC_SUMMARY.exists():
        return None
    m = re.search(r'^traffic_bytes_per_launch\s*=\s*(\d+)', TRAFFIC_SUMMARY.read_text(), re.M)
    return int(m.group(1)) if m else None


def sampler_call_us(device, calls=200):
    """Host wall time of one drop-in ``Sampler.sample`` call (B=1, logits on the GPU,
    including the parameter upload and the result download)."""
    import torch
    from klsample import Sampler, workloads
    w = workloads.make('latency_b1')
    logits = w.logits[0].to(device)
    s = Sampler(w.params[0], device=device)
    for _ in range(10):
        s.sample(logits)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(calls):
        s.sample(logits)
    return (time.perf_counter() - t0) * 1e6 / calls


def engine_step_us(device, batches=(1, 64, 256), calls=100):
    """Host wall time of one engine-shaped step (``klsample.engine.BatchedStep``): B
    requests with the headline row parameters, fp32 logits [B, 151936] on the GPU and
    2048-token device histories that grow by the sampled token each step.  One step is
    the uniforms, the parameter and range hand-over, the launch, the wait and the
    row-aligned result arrays with the stop flags (``BatchedStep.run``)."""
    import torch
    from klsample import Sampler, SamplingParams
    from klsample.engine import BatchedStep, DeviceHistory
    V, H = 151936, 2048
    g = torch.Generator(device=device).manual_seed(0)
    out = {}
    for B in batches:
        hist = DeviceHistory(device, V, capacity=B * (H + calls + 64), reserve=calls + 32)
        for b in range(B):
            hist.register(b, torch.randint(0, V, (H,), generator=g, device=device).cpu().numpy())
        samplers = [Sampler(SamplingParams(temperature=1.0, top_k=40, top_p=0.9, repetition_penalty=1.1,
                                           presence_penalty=0.5, frequency_penalty=0.3, seed=b), device=device)
                    for b in range(B)]
        logits = torch.randn(B, V, generator=g, device=device)
        step = BatchedStep(device, hist)
        rids = list(range(B))
        for _ in range(10):
            step.run(rids, samplers, logits)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(calls):
            step.run(rids, samplers, logits)
        out[f'b{B}'] = round((time.perf_counter() - t0) * 1e6 / calls, 1)
        del hist, step, logits
    return out


def lmhead_us(device, batches=(1, 8, 64, 256), calls=200):
    """Host wall per call (one synchronisation each) of the fused LM head + sampling call
    (``klsample_lmhead_run``) against torch's bf16 ``hidden @ weight.T`` followed by
    ``klsample_run``, at V = 151,936 and d = 1,024 (Qwen3-0.6B's LM head), greedy and
    top-k 50 rows, random bf16 weights and hidden states."""
    import numpy as np
    import torch
    from klsample import SamplingParams
    from klsample.lmhead import lmhead_sample
    from klsample.runner import runner_for
    V, d = 151936, 1024
    g = torch.Generator(device=device).manual_seed(0)
    weight = (torch.randn(V, d, generator=g, device=device) * (3.0 / d ** 0.5)).bfloat16()
    r = runner_for(device)

    def wall(fn):
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        torch.cuda.synchronize()
        return round((time.perf_counter() - t0) * 1e6 / calls, 1)

    out = {}
    for B in batches:
        hidden = torch.randn(B, d, generator=g, device=device).bfloat16()
        uni = np.full(B, 0.5, np.float32)
        for kind, p in (('greedy', SamplingParams()), ('top_k50', SamplingParams(temperature=0.8, top_k=50, seed=1))):
            params = [p] * B
            out[f'b{B}_{kind}'] = {
                'fused': wall(lambda: lmhead_sample(hidden, weight, params, None, uni)),
                'matmul_then_sample': wall(lambda: r.run((hidden @ weight.T).float(), params, None, uni, 0))}
    return out


# the other configurations of the sampling path, each timed at its own shape (device time
# per call, inputs resident): workload name, timed calls, warm-up calls
OTHER_CONFIGS = (
    ('cpu_reference_b8', 300, 30),
    ('mixed_b64', 60, 6),
    ('throughput_b256_v128256', 300, 30),
    ('tie_stress_b1024', 60, 6),
)


def per_config(device):
    """Device µs per call, rows/s and algorithmic GB/s of each other configuration."""
    out = {}
    for name, steps, warmup in OTHER_CONFIGS:
        r = Resident(name, device)
        _, d = timed_steps(r, steps, warmup)
        out[name] = {'batch': r.w.batch, 'vocab': r.w.vocab, 'logits': str(r.w.logits.dtype).replace('torch.', ''),
                     'device_us_per_call': round(d * 1e3, 2), 'rows_per_s': round(r.w.batch / (d * 1e-3), 1),
                     'alg_gbs': round(r.alg_bytes / (d * 1e-3) / 1e9, 1)}
        del r
    return out


def cpu_model():
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def cpu_baseline(seconds):
    """The oracle's faithful mode (torch CPU ops of serving/sampling.py:44-63 including
    torch.multinomial), one call per row of the headline batch, until ``seconds`` pass."""
    import torch
    from klsample import workloads
    from oracle.cpu_sampler import restated_sample
    w = workloads.make(HEADLINE)
    threads = torch.get_num_threads()
    gens = [torch.Generator().manual_seed(1000 + b) for b in range(w.batch)]
    restated_sample(w.logits[0], w.histories[0], w.params[0], generator=gens[0], diagnostics=False)  # warm
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        b = n % w.batch
        restated_sample(w.logits[b], w.histories[b], w.params[b], generator=gens[b], diagnostics=False)
        n += 1
    el = time.perf_counter() - t0
    # the same on one thread, for a quarter of the time
    torch.set_num_threads(1)
    n1 = 0
    t1 = time.perf_counter()
    while time.perf_counter() - t1 < seconds / 4:
        b = n1 % w.batch
        restated_sample(w.logits[b], w.histories[b], w.params[b], generator=gens[b], diagnostics=False)
        n1 += 1
    el1 = time.perf_counter() - t1
    torch.set_num_threads(threads)
    return {
        'value': round(n / el, 3), 'unit': 'rows/s', 'cores': threads, 'kind': 'port',
        'sample': (f'{n} row calls cycling over the B=256, V=151936 fp32 batch (T=1, top_k=40, top_p=0.9, '
                   f'three penalties, 2048-id histories), one restated Sampler.sample call per row with '
                   f'torch.multinomial, {threads} torch CPU threads, {el:.1f} s; {el / n * 1e3:.2f} ms/row; '
                   f'torch {torch.__version__}'),
        'cpu_model': cpu_model(),
        'host_cpus': os.cpu_count(),
        'one_thread': {'value': round(n1 / el1, 3), 'unit': 'rows/s',
                       'sample': f'{n1} row calls, 1 torch CPU thread, {el1:.1f} s; {el1 / n1 * 1e3:.2f} ms/row'},
    }


# ---- rocprofv3 CSV summaries ---------------------------------------------------------------

def _short(name):
    m = re.search(r'(\w+_kernel)<([^>]*)>', name)
    if m:
        return f'{m.group(1)}<{m.group(2).replace(" ", "")}>'
    m = re.search(r'(\w*copy\w*)', name)
    return (m.group(1) if m else name)[:60]


def _find(root, suffix):
    hits = sorted(Path(root).rglob(f'*{suffix}'))
    if not hits:
        raise SystemExit(f'no *{suffix} under {root}')
    return hits[-1]


def summarize_stats(root, command):
    """The rocprofv3 --stats table, plus per-(kernel, workgroups) durations from the trace."""
    path = _find(root, 'kernel_stats.csv')
    lines = ['# rocprofv3 kernel statistics', '', f'command: `{command}`', '',
             f'## {path.name}', '',
             '| kernel | calls | avg µs | min µs | max µs | total % |', '|---|---|---|---|---|---|']
    with open(path) as f:
        for r in csv.DictReader(f):
            lines.append(f"| {_short(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                         f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                         f"{float(r['Percentage']):.1f} |")
    trace = sorted(Path(root).rglob('*kernel_trace.csv'))
    if trace:
        groups, meta = {}, {}
        with open(trace[-1]) as f:
            for r in csv.DictReader(f):
                wgs = int(r['Grid_Size_X']) // max(int(r['Workgroup_Size_X']), 1)
                key = (_short(r['Kernel_Name']), wgs)
                groups.setdefault(key, []).append((int(r['End_Timestamp']) - int(r['Start_Timestamp'])) / 1e3)
                meta[key] = (r['VGPR_Count'], r['SGPR_Count'], r['LDS_Block_Size'], r['Scratch_Size'])
        lines += ['', f'## {trace[-1].name}: per kernel and grid', '',
                  '| kernel | workgroups | dispatches | avg µs | median µs | min µs | VGPR | SGPR | LDS B | scratch B |',
                  '|---|---|---|---|---|---|---|---|---|---|']
        for key, v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
            v = sorted(v)
            n = len(v)
            vg, sg, lds, scr = meta[key]
            lines.append(f'| {key[0]} | {key[1]} | {n} | {sum(v) / n:.2f} | {v[n // 2]:.2f} | {v[0]:.2f} | '
                         f'{vg} | {sg} | {lds} | {scr} |')
    print('\n'.join(lines))


def _counter_rows(root, counter):
    path = _find(root, 'counter_collection.csv')
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            if r.get('Counter_Name') == counter:
                rows.append((_short(r['Kernel_Name']), int(r['Grid_Size']), float(r['Counter_Value'])))
    return rows


def summarize_pmc(fetch_root, write_root, command_fetch, command_write):
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) per kernel, scaled by what the same
    counters read for the 1 GiB device copy of ``--profile-run`` (1 GiB read, 1 GiB
    written; the largest copy dispatch of the run)."""
    fetch, write = _counter_rows(fetch_root, 'FETCH_SIZE'), _counter_rows(write_root, 'WRITE_SIZE')
    kib = COPY_CALIBRATION_BYTES / 1024

    def calib(rows):
        copies = [v for k, g, v in rows if 'copy' in k.lower()]
        if not copies:
            raise SystemExit('no copy kernel in the counter output')
        return kib / max(copies), max(copies)

    ff, fcopy = calib(fetch)
    fw, wcopy = calib(write)

    def avg(rows):
        acc = {}
        for k, g, v in rows:
            if 'copy' not in k.lower():
                acc.setdefault((k, g), []).append(v)
        return {key: (sum(v) / len(v), len(v)) for key, v in acc.items()}

    fa, wa = avg(fetch), avg(write)
    lines = ['# rocprofv3 HBM byte counters', '', f'fetch command: `{command_fetch}`',
             f'write command: `{command_write}`', '',
             f'calibration: the {COPY_CALIBRATION_BYTES >> 20} MiB device copy reads FETCH_SIZE {fcopy:.0f} KiB '
             f'and WRITE_SIZE {wcopy:.0f} KiB for {kib:.0f} KiB moved each way, so FETCH_SIZE is scaled '
             f'by {ff:.4f} and WRITE_SIZE by {fw:.4f}', '',
             '| kernel | grid (threads) | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | scaled HBM bytes/launch |',
             '|---|---|---|---|---|---|']
    traffic = None
    for key in sorted(set(fa) | set(wa)):
        (fv, nf), (wv, nw) = fa.get(key, (0.0, 0)), wa.get(key, (0.0, 0))
        scaled = int(round((fv * ff + wv * fw) * 1024))
        lines.append(f'| {key[0]} | {key[1]} | {nf}/{nw} | {fv:.0f} | {wv:.0f} | {scaled} |')
        if key[0].startswith('scan_kernel<float,32'):   # the headline's (fp32, 32 elements per thread)
            traffic = scaled
    lines.append('')
    if traffic is not None:
        lines.append(f'traffic_bytes_per_launch = {traffic}')
    print('\n'.join(lines))


# ---- main ------------------------------------------------------------------------------------

def summarize_parity(path, command):
    """The parity counts the GPU tests log (one JSON line per comparison, written when
    KLSAMPLE_PARITY_LOG names a file) as a table per case."""
    rows = [json.loads(line) for line in Path(path).read_text().splitlines() if line.strip()]
    cols = ('rows', 'greedy', 'sampled', 'exact', 'tie_rows', 'margin_rows', 'cdf_rows', 'kept_differs',
            'boundary_mismatches', 'probs_rows', 'max_prob_rel', 'max_logprob_err', 'failures')
    agg = {}
    for r in rows:
        case = 'golden reference vectors' if r['case'].startswith('golden ') else r['case']
        a = agg.setdefault(case, dict.fromkeys(cols, 0))
        for c in cols:
            a[c] = max(a[c], r[c]) if c.startswith('max_') else a[c] + r[c]
    lines = ['# Parity counts of the GPU tests against the oracle', '', f'command: `{command}`', '',
             '* `exact`: rows whose token id equals the oracle\'s (stable tie order);',
             '* `tie_rows`: sampled rows with a value tie across the top-p cut (compared like any other);',
             '* `margin_rows` / `cdf_rows`: top-p mass or `u * Z` within 1e-6 (plus the reference\'s own fp32',
             '  normaliser error) of a boundary; `kept_differs`: margin rows whose kept count differs from the',
             '  reference\'s; `boundary_mismatches`: tokens that differ on such rows (each still in the kept set);',
             '* `max_prob_rel` / `max_logprob_err`: against the exact (float64) softmax / log-softmax.', '',
             '| case | ' + ' | '.join(cols) + ' |', '|---' * (len(cols) + 1) + '|']
    tot = dict.fromkeys(cols, 0)
    for case, a in agg.items():
        lines.append(f'| {case} | ' + ' | '.join(f'{a[c]:.3g}' if c.startswith('max_') else str(a[c]) for c in cols) + ' |')
        for c in cols:
            tot[c] = max(tot[c], a[c]) if c.startswith('max_') else tot[c] + a[c]
    lines.append('| **all** | ' + ' | '.join(f'{tot[c]:.3g}' if c.startswith('max_') else str(tot[c]) for c in cols) + ' |')
    print('\n'.join(lines))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=500)
    ap.add_argument('--warmup', type=int, default=50)
    ap.add_argument('--cpu-seconds', type=float, default=12.0)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--profile-run', action='store_true')
    ap.add_argument('--workload', default=None, help='workload of --profile-run (default: the headline)')
    ap.add_argument('--summarize-stats', metavar='DIR')
    ap.add_argument('--summarize-pmc', nargs=2, metavar=('FETCH_DIR', 'WRITE_DIR'))
    ap.add_argument('--summarize-parity', metavar='JSONL')
    ap.add_argument('--lmhead', action='store_true', help='fused LM head + sampling against matmul + sampling')
    ap.add_argument('--command', nargs='*', default=[])
    args = ap.parse_args()

    if args.summarize_stats:
        return summarize_stats(args.summarize_stats, ' '.join(args.command))
    if args.summarize_parity:
        return summarize_parity(args.summarize_parity, ' '.join(args.command))
    if args.summarize_pmc:
        cmds = ' '.join(args.command).split(' ;; ')
        return summarize_pmc(*args.summarize_pmc, cmds[0], cmds[-1])

    world = int(os.environ.get('WORLD_SIZE', '1'))
    if args.gpus != 1 or world != 1:
        print(f'bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}): '
              'the sampling path shards rows across GPUs with no exchange, so the per-GPU figure is '
              'the one-GPU run.', file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print('bench.py needs a ROCm GPU', file=sys.stderr)
        return 1
    device = torch.device('cuda', 0)
    torch.cuda.set_device(device)
    if args.lmhead:
        print(json.dumps({'lmhead_call_wall_us': lmhead_us(device)}), flush=True)
        return 0

    if args.profile_run:
        name = args.workload or HEADLINE
        res = Resident(name, device)
        for i in range(args.warmup + args.steps):
            res.launch(i)
        src = torch.empty(COPY_CALIBRATION_BYTES // 4, dtype=torch.float32, device=device).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f'profile run: {args.warmup + args.steps} steps of {name} and 3 copies of '
              f'{COPY_CALIBRATION_BYTES >> 20} MiB', flush=True)
        return 0

    res = Resident(HEADLINE, device)
    B = res.w.batch
    from klsample import workloads
    digests = ROOT / 'tests' / 'golden' / 'workload_digests.json'
    digest_ok = (json.loads(digests.read_text()).get(HEADLINE) == workloads.digest(res.w)) if digests.exists() else None
    ms_step, dev_ms = timed_steps(res, args.steps, args.warmup)
    first = res.token.clone()
    scan_ms, comb_ms = phase_times(res, min(args.steps, 200))
    torch.cuda.synchronize()
    consistent = bool(torch.equal(first, res.token))

    lat = {}
    for name, key in (('latency_b1', 'sampled'), ('latency_b1_greedy', 'greedy')):
        r1 = Resident(name, device)
        _, d = timed_steps(r1, 1000, 100)
        lat[key] = round(d * 1e3, 2)                      # mean over back-to-back calls
        groups = per_call_us(r1, 100, 10, 100)
        lat[key + '_median'] = round(groups[len(groups) // 2], 2)   # median of 100 groups of 10 calls
        lat[key + '_max'] = round(groups[-1], 2)
        del r1
    lat['sampler_call_wall'] = round(sampler_call_us(device), 1)
    engine_wall = engine_step_us(device)
    configs = per_config(device)

    achieved = res.alg_bytes / (scan_ms * 1e-3) / 1e9
    whole = res.alg_bytes / (dev_ms * 1e-3) / 1e9   # both kernels and the gaps between calls
    out = {
        'metric': METRIC,
        'value': round(B / (ms_step * 1e-3), 1),
        'unit': 'rows/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(ms_step, 5),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f32',
        'data': 'synthetic',
        'config': {'workload': HEADLINE, 'batch': B, 'vocab': res.w.vocab, 'logits': 'f32',
                   'temperature': 1.0, 'top_k': 40, 'top_p': 0.9, 'repetition_penalty': 1.1,
                   'presence_penalty': 0.5, 'frequency_penalty': 0.3, 'history': 2048,
                   'buffers': res.copies},
        'hbm_gbs': round(res.alg_bytes / (ms_step * 1e-3) / 1e9, 1),
        'device_us_per_step': round(dev_ms * 1e3, 2),
        'kernels_us': {'scan_kernel': round(scan_ms * 1e3, 2), 'row_kernel': round(comb_ms * 1e3, 2)},
        'b1_latency_us': lat,
        'engine_step_wall_us': engine_wall,
        'other_configs': configs,
        'roofline': {'bound': 'hbm', 'kernel': 'scan_kernel', 'achieved': round(achieved, 1), 'peak': PEAK_HBM_GBS,
                     'unit': 'GB/s', 'frac': round(achieved / PEAK_HBM_GBS, 4), 'traffic': read_traffic(),
                     'whole_call_achieved': round(whole, 1), 'whole_call_frac': round(whole / PEAK_HBM_GBS, 4)},
        'outputs_consistent': consistent,
        'workload_sha256_ok': digest_ok,
    }
    if not args.no_cpu_baseline:
        out['cpu_baseline'] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == '__main__':
    sys.exit(main())
