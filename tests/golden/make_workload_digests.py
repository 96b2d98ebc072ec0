"""Write ``workload_digests.json``: the SHA-256 of every configured workload (logits,
uniforms, histories, parameters) as generated on this machine.  The tests and the bench
compare fresh generations against it, on any machine, to catch generator drift.

    python tests/golden/make_workload_digests.py
"""
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / 'gpu-kernel-lab_amd'))

from klsample import workloads  # noqa: E402


def main():
    out = {name: workloads.digest(workloads.make(name)) for name in workloads.NAMES}
    (HERE / 'workload_digests.json').write_text(json.dumps(out, indent=1, sort_keys=True) + '\n')
    print(json.dumps(out, indent=1))


if __name__ == '__main__':
    main()
