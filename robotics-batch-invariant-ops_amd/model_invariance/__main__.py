"""python -m model_invariance [--adapter synthetic_vla] [--preset small|vla] [--batch-sizes 1,2,...]
[--invariant-ops] [--seed 0] [--output report.json]: run the investigation and print its
summary (one line per composition and batch size)."""

from __future__ import annotations

import argparse

from .adapters import ADAPTERS
from .harness import DEFAULT_BATCH_SIZES, run_investigation


def main(argv=None) -> int:
    p = argparse.ArgumentParser(prog="python -m model_invariance")
    p.add_argument("--adapter", choices=sorted(ADAPTERS), default="synthetic_vla")
    p.add_argument("--preset", default="small", help="synthetic_vla sizes: small or vla")
    p.add_argument("--batch-sizes", default=",".join(map(str, DEFAULT_BATCH_SIZES)))
    p.add_argument("--invariant-ops", action="store_true", help="run under set_batch_invariant_mode()")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--output", default=None)
    args = p.parse_args(argv)
    sizes = [int(s) for s in args.batch_sizes.split(",") if s]
    adapter_cls = ADAPTERS[args.adapter]
    adapter = adapter_cls.preset(args.preset) if hasattr(adapter_cls, "preset") else adapter_cls()
    report = run_investigation(adapter, batch_sizes=sizes, invariant_ops=args.invariant_ops,
                               seed=args.seed, output_path=args.output)
    print(f"model={report['model']} invariant_ops={report['batch_invariant_ops']} "
          f"repeatable={report['repeatability']['exact']} end_to_end_exact={report['end_to_end_exact']}")
    for name, results in report["composition_results"].items():
        for r in results:
            print(f"  {name:9s} B={r['batch_size']:3d} {r['status']}")
    return 0 if report["end_to_end_exact"] else 1


if __name__ == "__main__":
    raise SystemExit(main())
