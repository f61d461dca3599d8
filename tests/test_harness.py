"""Model-level invariance harness (reference test_investigation_harness.py:1-70 and
scripts/model_invariance/harness.py): report schema, diagnostics, OOM stop, and, on the GPU, a
synthetic action-expert model that is bitwise batch invariant end to end under the mode."""

from __future__ import annotations

import json

import pytest
import torch

from model_invariance import compare_outputs, run_investigation
from model_invariance.harness import NOT_REPEATABLE, first_sample, flatten_outputs, stack_samples, tensor_sha256


class SyntheticAdapter:
    """Identity model over two-element samples; optionally adds the batch size (a model whose
    output depends on the batch)."""

    name = "synthetic"

    def __init__(self, batch_dependent: bool = False, oom_from: int | None = None, flaky: bool = False):
        self.batch_dependent = batch_dependent
        self.oom_from = oom_from
        self.flaky = flaky
        self.calls = 0

    def load_model(self):
        return torch.nn.Identity()

    def load_example_inputs(self, count: int):
        return [{"x": torch.tensor([float(i), 2.0])} for i in range(count)]

    def run_model(self, model, batch):
        self.calls += 1
        x = batch["x"]
        if self.oom_from is not None and x.shape[0] >= self.oom_from:
            raise torch.cuda.OutOfMemoryError("HIP out of memory. Tried to allocate 2.00 GiB")
        out = model(x)
        if self.batch_dependent:
            out = out + out.shape[0]
        if self.flaky:
            out = out + self.calls
        return {"actions": out, "trajectory": (out[:, None, :],)}

    def extract_robot_output(self, output):
        return output


def test_compare_outputs_reports_first_difference_and_hashes():
    [d] = compare_outputs({"actions": torch.tensor([[1.0, 2.0]])}, {"actions": torch.tensor([[1.0, 3.0]])})
    assert not d.exact
    assert d.differing_elements == 1
    assert d.first_differing_index == (0, 1)
    assert d.max_abs_difference == 1.0 and d.mean_abs_difference == 0.5
    assert d.reference_hash != d.candidate_hash
    [same] = compare_outputs({"a": torch.ones(3)}, {"a": torch.ones(3)})
    assert same.exact and same.differing_elements == 0 and same.first_differing_index is None
    assert same.reference_hash == same.candidate_hash == tensor_sha256(torch.ones(3))


def test_compare_outputs_metadata_and_structure():
    [d] = compare_outputs({"a": torch.ones(2)}, {"a": torch.ones(3)})
    assert not d.exact and d.differing_elements is None and d.candidate_shape == (3,)
    [d] = compare_outputs({"a": torch.ones(2)}, {"a": torch.ones(2, dtype=torch.float64)})
    assert not d.exact
    with pytest.raises(ValueError):
        compare_outputs({"a": torch.ones(2)}, {"b": torch.ones(2)})
    with pytest.raises(TypeError):
        flatten_outputs({"a": object()})
    # integer outputs: exact / count without magnitudes
    [d] = compare_outputs({"i": torch.tensor([1, 2])}, {"i": torch.tensor([1, 5])})
    assert d.differing_elements == 1 and d.max_abs_difference is None


def test_flatten_paths_and_first_sample():
    out = {"b": (torch.zeros(2, 3), [torch.ones(2)]), "a": torch.tensor(5.0)}
    assert list(flatten_outputs(out)) == ["output.a", "output.b[0]", "output.b[1][0]"]
    s = first_sample(out)
    assert s["b"][0].shape == (1, 3) and s["b"][1][0].shape == (1,) and s["a"].ndim == 0


def test_stack_samples_rules():
    batch = stack_samples([{"x": torch.zeros(2), "k": 3}, {"x": torch.ones(2), "k": 3}])
    assert batch["x"].shape == (2, 2) and batch["k"] == 3
    with pytest.raises(ValueError):
        stack_samples([{"k": 1}, {"k": 2}])


def test_investigation_covers_duplicate_and_unrelated_compositions(tmp_path):
    output = tmp_path / "result.json"
    report = run_investigation(SyntheticAdapter(), batch_sizes=(1, 2, 3, 5), output_path=output)
    assert report["repeatability"]["exact"]
    assert report["end_to_end_exact"]
    assert report["maximum_tested_batch"] == 5
    assert [r["batch_size"] for r in report["composition_results"]["duplicate"]] == [1, 2, 3, 5]
    assert [r["batch_size"] for r in report["composition_results"]["unrelated"]] == [1, 2, 3, 5]
    assert json.loads(output.read_text())["end_to_end_exact"]


def test_investigation_detects_batch_dependent_final_output():
    report = run_investigation(SyntheticAdapter(batch_dependent=True), batch_sizes=(1, 2, 3))
    assert report["repeatability"]["exact"]
    assert not report["end_to_end_exact"]
    assert report["composition_results"]["duplicate"][0]["status"] == "PASS"
    assert report["composition_results"]["duplicate"][1]["status"] == "FAIL"
    tensor = report["composition_results"]["unrelated"][2]["tensors"][0]
    assert tensor["differing_elements"] == 2


def test_investigation_stops_a_composition_at_out_of_memory():
    report = run_investigation(SyntheticAdapter(oom_from=4), batch_sizes=(1, 2, 4, 8))
    for name in ("duplicate", "unrelated"):
        results = report["composition_results"][name]
        assert [r["status"] for r in results] == ["PASS", "PASS", "OOM"]
    assert report["maximum_tested_batch"] == 2
    assert report["end_to_end_exact"]


def test_investigation_reports_non_repeatable_model():
    report = run_investigation(SyntheticAdapter(flaky=True), batch_sizes=(1, 2))
    assert not report["repeatability"]["exact"]
    assert report["failure"] == NOT_REPEATABLE
    assert report["composition_results"]["duplicate"] == []
    assert not report["end_to_end_exact"]


def test_investigation_rejects_bad_batch_sizes():
    with pytest.raises(ValueError):
        run_investigation(SyntheticAdapter(), batch_sizes=(2, 3))


@pytest.mark.gpu
def test_synthetic_vla_is_batch_invariant_end_to_end_under_the_mode(tmp_path):
    from model_invariance.adapters import SyntheticVLAAdapter

    report = run_investigation(SyntheticVLAAdapter(), batch_sizes=(1, 2, 3, 5, 8, 17), invariant_ops=True,
                               output_path=tmp_path / "vla.json")
    assert report["repeatability"]["exact"]
    bad = [(name, r["batch_size"]) for name, rs in report["composition_results"].items()
           for r in rs if r["status"] != "PASS"]
    assert not bad, f"not batch invariant: {bad}"
    assert report["end_to_end_exact"]
    assert report["native_library"] and "libbiops.so" in report["native_library"]
