"""Model-level batch-invariance investigation: does a whole model's output for one sample keep
its bits when the sample shares a batch with copies of itself or with unrelated samples?

Mirrors the reference harness (scripts/model_invariance/harness.py:1-312): the same adapter
protocol (load_model / load_example_inputs / run_model / extract_robot_output, optional
compose_batch and reset_model), the same report schema (repeatability, duplicate and unrelated
compositions per batch size, per-tensor diagnostics with sha256 of the raw bytes, OOM stop,
``end_to_end_exact``) so reports of both builds can be diffed.

On a ROCm GPU the comparison runs on the device (one elementwise ``!=`` and its reductions per
tensor) and only the bytes to hash cross to the host.  Out-of-memory is recognised from
torch's ``OutOfMemoryError`` or the HIP / CUDA runtime message, ends that composition and frees
the cache.  The report also records which kernel library answered (``native_library``).
"""

from __future__ import annotations

import contextlib
import dataclasses
import hashlib
import json
import random
from collections.abc import Callable, Mapping, Sequence
from pathlib import Path
from typing import Any, Protocol, runtime_checkable

import numpy as np
import torch

from batch_invariant_ops import set_batch_invariant_mode

# Batch sizes of the reference's sweep (harness.py:24): small primes, powers of two and their
# neighbours, so that tile-boundary effects show up.
DEFAULT_BATCH_SIZES = (1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 32, 33, 64)


@runtime_checkable
class ModelAdapter(Protocol):
    """What the harness needs from a model integration (reference harness.py:27-39)."""

    name: str

    def load_model(self) -> Any: ...

    def load_example_inputs(self, count: int) -> Sequence[Any]: ...

    def run_model(self, model: Any, batch: Any) -> Any: ...

    def extract_robot_output(self, output: Any) -> Any: ...


@dataclasses.dataclass(frozen=True)
class TensorDifference:
    """Diagnostics of one output tensor (field names of reference harness.py:42-54)."""

    path: str
    reference_shape: tuple[int, ...]
    candidate_shape: tuple[int, ...]
    dtype: str
    exact: bool
    differing_elements: int | None
    max_abs_difference: float | None
    mean_abs_difference: float | None
    first_differing_index: tuple[int, ...] | None
    reference_hash: str
    candidate_hash: str


def seed_everything(seed: int) -> None:
    """Reset Python, NumPy and torch (host and every device) generators."""
    random.seed(seed)
    np.random.seed(seed)
    torch.manual_seed(seed)  # also seeds every visible GPU generator


def tensor_sha256(tensor: torch.Tensor) -> str:
    """sha256 of the tensor's raw bytes in row-major order (dtype-exact, -0.0 != 0.0)."""
    host = tensor.detach().contiguous().cpu()
    return hashlib.sha256(host.view(torch.uint8).numpy().tobytes()).hexdigest()


def flatten_outputs(value: Any, path: str = "output") -> dict[str, torch.Tensor]:
    """Tensors of a nested output keyed by access path: ``output.key``, ``output[i]``.  Mapping
    keys are visited in sorted order so the two sides line up."""
    if isinstance(value, torch.Tensor):
        return {path: value}
    found: dict[str, torch.Tensor] = {}
    if isinstance(value, Mapping):
        for key in sorted(value, key=str):
            found.update(flatten_outputs(value[key], f"{path}.{key}"))
        return found
    if isinstance(value, (tuple, list)):
        for i, item in enumerate(value):
            found.update(flatten_outputs(item, f"{path}[{i}]"))
        return found
    raise TypeError(f"{path} contains unsupported output type {type(value).__name__}")


def first_sample(value: Any) -> Any:
    """Sample 0 of every tensor in a nested output (leading dim kept; 0-d tensors as they are)."""
    if isinstance(value, torch.Tensor):
        return value if value.ndim == 0 else value[:1]
    if isinstance(value, Mapping):
        return type(value)((k, first_sample(v)) for k, v in value.items())
    if isinstance(value, tuple):
        return tuple(first_sample(v) for v in value)
    if isinstance(value, list):
        return [first_sample(v) for v in value]
    raise TypeError(f"unsupported output type {type(value).__name__}")


def _difference(path: str, ref: torch.Tensor, cand: torch.Tensor) -> TensorDifference:
    same_meta = ref.shape == cand.shape and ref.dtype == cand.dtype
    count = max_abs = mean_abs = first = None
    exact = False
    if same_meta:
        if cand.device != ref.device:
            cand = cand.to(ref.device)
        # value comparison, as torch.equal (a NaN never matches); the hashes compare raw bytes
        differs = ref != cand
        count = int(differs.sum().item())
        exact = count == 0
        if count:
            first = tuple(int(i) for i in torch.nonzero(differs)[0].tolist())
        if ref.is_floating_point() or ref.is_complex():
            if ref.numel():
                gap = (ref - cand).abs().float()
                max_abs = float(gap.max().item())
                mean_abs = float(gap.mean().item())
            else:
                max_abs = mean_abs = 0.0
    return TensorDifference(
        path=path,
        reference_shape=tuple(ref.shape),
        candidate_shape=tuple(cand.shape),
        dtype=str(ref.dtype),
        exact=exact,
        differing_elements=count,
        max_abs_difference=max_abs,
        mean_abs_difference=mean_abs,
        first_differing_index=first,
        reference_hash=tensor_sha256(ref),
        candidate_hash=tensor_sha256(cand),
    )


def compare_outputs(reference: Any, candidate: Any) -> list[TensorDifference]:
    """Per-tensor diagnostics of two outputs with the same structure (ValueError otherwise)."""
    ref = flatten_outputs(reference)
    cand = flatten_outputs(candidate)
    if ref.keys() != cand.keys():
        raise ValueError(f"output structures differ: reference={sorted(ref)}, candidate={sorted(cand)}")
    return [_difference(path, ref[path], cand[path]) for path in ref]


def stack_samples(samples: Sequence[Any]) -> Any:
    """Default batch composition: stack tensors on a new leading dim, recursively through
    mappings / tuples / lists; plain metadata must agree across samples."""
    head = samples[0]
    if isinstance(head, torch.Tensor):
        return torch.stack(list(samples))
    if isinstance(head, Mapping):
        return type(head)((k, stack_samples([s[k] for s in samples])) for k in head)
    if isinstance(head, (tuple, list)):
        parts = [stack_samples([s[i] for s in samples]) for i in range(len(head))]
        return tuple(parts) if isinstance(head, tuple) else parts
    if isinstance(head, (bool, int, float, str)):
        if any(s != head for s in samples):
            raise ValueError("non-tensor metadata differs; provide adapter.compose_batch")
        return head
    raise TypeError(f"cannot batch {type(head).__name__}; provide adapter.compose_batch")


def is_out_of_memory(error: BaseException) -> bool:
    """True for device out-of-memory errors (torch's class or the runtime's message)."""
    oom_type = getattr(torch.cuda, "OutOfMemoryError", None)
    if oom_type is not None and isinstance(error, oom_type):
        return True
    return "out of memory" in str(error).lower()


def _native_library() -> str | None:
    try:
        from batch_invariant_ops import _native

        return f"{_native.lib_version()} ({_native.library_path().name})"
    except Exception:  # the library is optional for a stock-kernel investigation
        return None


class _Runner:
    """One adapter + model: composes batches and runs them from a fixed seed."""

    def __init__(self, adapter: ModelAdapter, model: Any, seed: int):
        self.adapter, self.model, self.seed = adapter, model, seed
        self.compose: Callable[[Sequence[Any]], Any] = getattr(adapter, "compose_batch", stack_samples)
        self.reset = getattr(adapter, "reset_model", None)

    def __call__(self, samples: Sequence[Any]) -> Any:
        batch = self.compose(samples)
        seed_everything(self.seed)
        if self.reset is not None:
            self.reset(self.model)
        with torch.inference_mode():
            return self.adapter.extract_robot_output(self.adapter.run_model(self.model, batch))


def _record(diffs: list[TensorDifference]) -> dict[str, Any]:
    return {"exact": all(d.exact for d in diffs), "tensors": [dataclasses.asdict(d) for d in diffs]}


def run_investigation(
    adapter: ModelAdapter,
    *,
    batch_sizes: Sequence[int] = DEFAULT_BATCH_SIZES,
    invariant_ops: bool = False,
    seed: int = 0,
    output_path: str | Path | None = None,
) -> dict[str, Any]:
    """Repeatability, then sample 0 of duplicate and unrelated batches of every size against
    the batch-of-one output (reference harness.py:222-312).  Returns the report and writes it
    as JSON to ``output_path`` when given."""
    sizes = tuple(sorted(set(int(b) for b in batch_sizes)))
    if not sizes or sizes[0] != 1:
        raise ValueError("batch_sizes must be positive and include 1")

    seed_everything(seed)
    model = adapter.load_model()
    if hasattr(model, "eval"):
        model.eval()
    examples = list(adapter.load_example_inputs(sizes[-1]))
    if not examples:
        raise ValueError("adapter returned no example inputs")
    if sizes[-1] > 1 and len(examples) < 2:
        raise ValueError("unrelated composition requires at least two example inputs")
    target, others = examples[0], examples[1:]

    report: dict[str, Any] = {
        "model": adapter.name,
        "batch_invariant_ops": invariant_ops,
        "seed": seed,
        "requested_batch_sizes": list(sizes),
        "repeatability": None,
        "composition_results": {"duplicate": [], "unrelated": []},
        "maximum_tested_batch": None,
        "end_to_end_exact": False,
        "native_library": _native_library() if invariant_ops else None,
    }
    run = _Runner(adapter, model, seed)
    compositions = {
        "duplicate": lambda n: [target] * n,
        "unrelated": lambda n: [target] + [others[i % len(others)] for i in range(n - 1)],
    }

    with set_batch_invariant_mode() if invariant_ops else contextlib.nullcontext():
        reference = run([target])
        report["repeatability"] = _record(compare_outputs(reference, run([target])))
        if not report["repeatability"]["exact"]:
            report["failure"] = "same-batch inference is not repeatable"
        else:
            largest = 1
            for name, samples_of in compositions.items():
                results = report["composition_results"][name]
                for n in sizes:
                    try:
                        candidate = run(samples_of(n))
                    except RuntimeError as error:
                        if not is_out_of_memory(error):
                            raise
                        if torch.cuda.is_available():
                            torch.cuda.empty_cache()
                        results.append({"batch_size": n, "status": "OOM"})
                        break
                    diffs = compare_outputs(reference, first_sample(candidate))
                    entry = {"batch_size": n, "status": "PASS" if all(d.exact for d in diffs) else "FAIL"}
                    entry.update(_record(diffs))
                    results.append(entry)
                    largest = max(largest, n)
            report["maximum_tested_batch"] = largest
            ran = [r for rs in report["composition_results"].values() for r in rs if r["status"] != "OOM"]
            report["end_to_end_exact"] = bool(ran) and all(r["status"] == "PASS" for r in ran)

    if output_path is not None:
        out = Path(output_path)
        out.parent.mkdir(parents=True, exist_ok=True)
        out.write_text(json.dumps(report, indent=2) + "\n")
    return report
