"""Model-level batch-invariance investigation.

Question asked: does the output a model produces for one sample keep its exact bits when that
sample is run inside a larger batch, either next to copies of itself ("duplicate") or next to
other samples ("unrelated")?

Interchange format shared with the reference harness (scripts/model_invariance/harness.py:1-312),
so that the two builds' reports can be diffed: the adapter methods (``load_model``,
``load_example_inputs``, ``run_model``, ``extract_robot_output``, optional ``compose_batch`` /
``reset_model``), the batch-size sweep, the report keys and the per-tensor record fields.

How this implementation works:

* An output is indexed once into ``(path, tensor)`` leaves by an explicit-stack walk; mapping
  keys are visited in sorted order and paths read ``output.key`` / ``output[i]``.
* A comparison reduces each tensor pair on its own device into four numbers (differing count,
  flat position of the first difference, max and mean absolute difference) that cross to the
  host in one transfer; only the raw bytes for the sha256 digests follow.
* Batches are composed by zipping the samples' structures leaf by leaf (``torch.stack`` for
  tensors; plain values must agree).
* The sweep is a list of trials (composition, batch size).  A trial that runs out of device
  memory closes its composition: the larger sizes of that composition are not attempted.
"""

from __future__ import annotations

import contextlib
import dataclasses
import hashlib
import json
import random
from collections.abc import Callable, Iterator, Mapping, Sequence
from pathlib import Path
from typing import Any, Protocol, runtime_checkable

import numpy as np
import torch

from batch_invariant_ops import set_batch_invariant_mode

# The sweep: small primes, powers of two and their neighbours, where tile edges show up.
DEFAULT_BATCH_SIZES = (1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 32, 33, 64)

COMPOSITIONS = ("duplicate", "unrelated")
NOT_REPEATABLE = "the batch-of-one output changes between two identical runs"


@runtime_checkable
class ModelAdapter(Protocol):
    """Model integration used by the investigation (method names are the interchange format)."""

    name: str

    def load_model(self) -> Any: ...

    def load_example_inputs(self, count: int) -> Sequence[Any]: ...

    def run_model(self, model: Any, batch: Any) -> Any: ...

    def extract_robot_output(self, output: Any) -> Any: ...


@dataclasses.dataclass(frozen=True)
class TensorDifference:
    """Record of one output tensor (field names are the interchange format)."""

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
    """Put Python's, NumPy's and torch's generators (host and all devices) in a known state."""
    random.seed(seed)
    np.random.seed(seed)
    torch.manual_seed(seed)  # torch seeds every visible device generator as well


def tensor_sha256(tensor: torch.Tensor) -> str:
    """Digest of the tensor's storage bytes in row-major order (so -0.0 and 0.0 differ)."""
    data = tensor.detach().contiguous().cpu().reshape(-1).view(torch.uint8)
    return hashlib.sha256(memoryview(data.numpy())).hexdigest()


# ----------------------------------------------------------------- output structure ----
def _children(value: Any, path: str) -> list[tuple[str, Any]] | None:
    """The (path, child) pairs of a container, None for a leaf tensor; TypeError otherwise."""
    if isinstance(value, torch.Tensor):
        return None
    if isinstance(value, Mapping):
        return [(f"{path}.{key}", value[key]) for key in sorted(value, key=str)]
    if isinstance(value, (list, tuple)):
        return [(f"{path}[{i}]", item) for i, item in enumerate(value)]
    raise TypeError(f"{path}: a {type(value).__name__} is not a tensor, mapping or sequence")


def flatten_outputs(value: Any, path: str = "output") -> dict[str, torch.Tensor]:
    """Every tensor of a nested output, keyed by its access path, in canonical order."""
    leaves: dict[str, torch.Tensor] = {}
    pending: list[tuple[str, Any]] = [(path, value)]
    while pending:
        where, node = pending.pop()
        kids = _children(node, where)
        if kids is None:
            leaves[where] = node
        else:
            pending.extend(reversed(kids))  # popped in forward order
    return leaves


def _rebuild(value: Any, on_tensor: Callable[[torch.Tensor], torch.Tensor]) -> Any:
    """The same container structure with ``on_tensor`` applied to every tensor."""
    if isinstance(value, torch.Tensor):
        return on_tensor(value)
    if isinstance(value, Mapping):
        return type(value)((key, _rebuild(item, on_tensor)) for key, item in value.items())
    if isinstance(value, (list, tuple)):
        items = [_rebuild(item, on_tensor) for item in value]
        return items if isinstance(value, list) else tuple(items)
    raise TypeError(f"a {type(value).__name__} is not a tensor, mapping or sequence")


def first_sample(value: Any) -> Any:
    """Sample 0 of a batched output: every tensor cut to its first leading index (dim kept);
    0-d tensors pass through."""
    return _rebuild(value, lambda t: t if t.ndim == 0 else t.narrow(0, 0, 1))


def stack_samples(samples: Sequence[Any]) -> Any:
    """Default ``compose_batch``: zip the samples' structures; tensors are stacked on a new
    leading dimension and plain values (bool / int / float / str) must be equal."""
    head = samples[0]
    if isinstance(head, torch.Tensor):
        return torch.stack(list(samples))
    if isinstance(head, Mapping):
        return type(head)((key, stack_samples([s[key] for s in samples])) for key in head)
    if isinstance(head, (list, tuple)):
        zipped = [stack_samples(column) for column in zip(*samples)]
        return zipped if isinstance(head, list) else tuple(zipped)
    if isinstance(head, (bool, int, float, str)):
        unequal = sorted({repr(s) for s in samples if s != head})
        if unequal:
            raise ValueError(
                f"samples carry different plain values ({head!r} vs {', '.join(unequal)}); "
                "the adapter must define compose_batch to batch them")
        return head
    raise TypeError(f"no default way to batch a {type(head).__name__}; the adapter must define compose_batch")


# ------------------------------------------------------------------------ comparison ----
def _stats(ref: torch.Tensor, cand: torch.Tensor) -> tuple[int, int, float | None, float | None]:
    """(differing count, flat index of the first difference or -1, max |diff|, mean |diff|),
    computed on the tensors' device and read back in one transfer.  Differences are by value,
    so NaN never equals NaN (the digests compare raw bytes)."""
    n = ref.numel()
    ne = (ref != cand).reshape(-1)
    positions = torch.arange(n, device=ne.device, dtype=torch.int64)
    first = torch.where(ne, positions, torch.full_like(positions, n)).amin() if n else ne.new_zeros((), dtype=torch.int64)
    parts = [ne.sum(dtype=torch.int64).double(), first.double()]
    magnitudes = ref.is_floating_point() or ref.is_complex()
    if magnitudes:
        if n:
            # sum / n rather than mean(): the comparison may run under the batch-invariant
            # mode, whose mean override has no float64 kernel
            gap = (ref - cand).abs().reshape(-1).double()
            parts += [gap.max(), gap.sum() / n]
        else:
            parts += [torch.zeros((), dtype=torch.float64, device=ne.device)] * 2
    values = torch.stack([p.to(ne.device) for p in parts]).cpu().tolist()
    count = int(values[0])
    first_flat = int(values[1]) if count else -1
    if not magnitudes:
        return count, first_flat, None, None
    return count, first_flat, float(values[2]), float(values[3])


def _difference(path: str, ref: torch.Tensor, cand: torch.Tensor) -> TensorDifference:
    count = first = max_abs = mean_abs = None
    if ref.shape == cand.shape and ref.dtype == cand.dtype:
        cand = cand.to(ref.device)
        count, flat, max_abs, mean_abs = _stats(ref, cand)
        if count:
            first = tuple(int(i) for i in np.unravel_index(flat, tuple(ref.shape)))
    return TensorDifference(
        path=path,
        reference_shape=tuple(ref.shape),
        candidate_shape=tuple(cand.shape),
        dtype=str(ref.dtype),
        exact=count == 0,
        differing_elements=count,
        max_abs_difference=max_abs,
        mean_abs_difference=mean_abs,
        first_differing_index=first,
        reference_hash=tensor_sha256(ref),
        candidate_hash=tensor_sha256(cand),
    )


def compare_outputs(reference: Any, candidate: Any) -> list[TensorDifference]:
    """One record per output tensor; ValueError when the two outputs hold different paths."""
    ref, cand = flatten_outputs(reference), flatten_outputs(candidate)
    if ref.keys() != cand.keys():
        only_ref = sorted(set(ref) - set(cand))
        only_cand = sorted(set(cand) - set(ref))
        raise ValueError(f"outputs hold different tensors: only in reference {only_ref}, "
                         f"only in candidate {only_cand}")
    return [_difference(path, tensor, cand[path]) for path, tensor in ref.items()]


def _summary(records: list[TensorDifference]) -> dict[str, Any]:
    return {"exact": all(r.exact for r in records), "tensors": [dataclasses.asdict(r) for r in records]}


def is_out_of_memory(error: BaseException) -> bool:
    """A device allocation failure: torch's OutOfMemoryError or the runtime's message."""
    oom_types = tuple(t for t in (getattr(torch, "OutOfMemoryError", None),
                                  getattr(torch.cuda, "OutOfMemoryError", None)) if t is not None)
    return isinstance(error, oom_types) or "out of memory" in str(error).lower()


def _native_library() -> str | None:
    """Which kernel library answered (None when it cannot be loaded)."""
    try:
        from batch_invariant_ops import _native

        return f"{_native.lib_version()} ({_native.library_path().name})"
    except Exception:  # a stock-kernel investigation does not need the library
        return None


# --------------------------------------------------------------------- investigation ----
@dataclasses.dataclass
class _Model:
    """A loaded model and how to run a list of samples through it from a fixed seed."""

    adapter: ModelAdapter
    model: Any
    seed: int

    def infer(self, samples: Sequence[Any]) -> Any:
        compose = getattr(self.adapter, "compose_batch", None) or stack_samples
        batch = compose(samples)
        seed_everything(self.seed)
        reset = getattr(self.adapter, "reset_model", None)
        if reset is not None:
            reset(self.model)
        with torch.inference_mode():
            raw = self.adapter.run_model(self.model, batch)
        return self.adapter.extract_robot_output(raw)


@dataclasses.dataclass(frozen=True)
class _Trial:
    composition: str
    batch_size: int
    samples: tuple


def _trials(sizes: Sequence[int], target: Any, others: Sequence[Any]) -> Iterator[_Trial]:
    """Duplicate batches (the target n times), then unrelated ones (the target followed by the
    other examples in turn), each over every size in increasing order."""
    for n in sizes:
        yield _Trial("duplicate", n, (target,) * n)
    for n in sizes:
        yield _Trial("unrelated", n, (target, *(others[i % len(others)] for i in range(n - 1))))


def _checked_sizes(batch_sizes: Sequence[int]) -> tuple[int, ...]:
    sizes = tuple(sorted({int(b) for b in batch_sizes}))
    if not sizes or sizes[0] < 1 or 1 not in sizes:
        raise ValueError(f"batch sizes {list(batch_sizes)} must all be >= 1 and contain the reference size 1")
    return sizes


def run_investigation(
    adapter: ModelAdapter,
    *,
    batch_sizes: Sequence[int] = DEFAULT_BATCH_SIZES,
    invariant_ops: bool = False,
    seed: int = 0,
    output_path: str | Path | None = None,
) -> dict[str, Any]:
    """Run the sweep and return the report (also written as JSON to ``output_path``).

    The batch-of-one output must first be repeatable; every trial then compares sample 0 of
    its output with it.  ``end_to_end_exact`` is true when every trial that ran matched.
    Interchange format: the reference's run_investigation (harness.py:222-312).
    """
    sizes = _checked_sizes(batch_sizes)
    seed_everything(seed)
    model = adapter.load_model()
    if hasattr(model, "eval"):
        model.eval()
    examples = list(adapter.load_example_inputs(sizes[-1]))
    if not examples:
        raise ValueError(f"adapter {adapter.name!r} produced no example inputs")
    if sizes[-1] > 1 and len(examples) < 2:
        raise ValueError(f"adapter {adapter.name!r} produced one example; unrelated batches need two or more")
    runner = _Model(adapter, model, seed)

    report: dict[str, Any] = {
        "model": adapter.name,
        "batch_invariant_ops": invariant_ops,
        "seed": seed,
        "requested_batch_sizes": list(sizes),
        "repeatability": None,
        "composition_results": {name: [] for name in COMPOSITIONS},
        "maximum_tested_batch": None,
        "end_to_end_exact": False,
        "native_library": _native_library() if invariant_ops else None,
    }
    mode = set_batch_invariant_mode() if invariant_ops else contextlib.nullcontext()
    with mode:
        baseline = runner.infer([examples[0]])
        report["repeatability"] = _summary(compare_outputs(baseline, runner.infer([examples[0]])))
        if report["repeatability"]["exact"]:
            _sweep(runner, baseline, sizes, examples, report)
        else:
            report["failure"] = NOT_REPEATABLE

    if output_path is not None:
        path = Path(output_path)
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(json.dumps(report, indent=2) + "\n")
    return report


def _sweep(runner: _Model, baseline: Any, sizes, examples, report: dict[str, Any]) -> None:
    closed: set[str] = set()  # compositions stopped by an out-of-memory trial
    results = report["composition_results"]
    for trial in _trials(sizes, examples[0], examples[1:]):
        if trial.composition in closed:
            continue
        try:
            output = runner.infer(trial.samples)
        except RuntimeError as error:
            if not is_out_of_memory(error):
                raise
            closed.add(trial.composition)
            if torch.cuda.is_available():
                torch.cuda.empty_cache()
            results[trial.composition].append({"batch_size": trial.batch_size, "status": "OOM"})
            continue
        summary = _summary(compare_outputs(baseline, first_sample(output)))
        results[trial.composition].append(
            {"batch_size": trial.batch_size, "status": "PASS" if summary["exact"] else "FAIL", **summary})
    ran = [r for rs in results.values() for r in rs if r["status"] != "OOM"]
    report["maximum_tested_batch"] = max((r["batch_size"] for r in ran), default=1)
    report["end_to_end_exact"] = bool(ran) and all(r["status"] == "PASS" for r in ran)


__all__ = [
    "COMPOSITIONS",
    "DEFAULT_BATCH_SIZES",
    "ModelAdapter",
    "NOT_REPEATABLE",
    "TensorDifference",
    "compare_outputs",
    "first_sample",
    "flatten_outputs",
    "is_out_of_memory",
    "run_investigation",
    "seed_everything",
    "stack_samples",
    "tensor_sha256",
]
