"""The tuning file (mhc_mlx/metal.py:21-36, scripts/tune.py): loading, precedence and the
reference's integer entries (CPU)."""

import json
import os

import pytest

from mhc_mlx_amd import tuning
from mhc_mlx_amd.metal import _get_tuned_tpg

KNOB_ENVS = sorted({env for env, _ in tuning.KNOBS.values()})


@pytest.fixture
def clean_env(monkeypatch):
    for env in KNOB_ENVS:
        monkeypatch.delenv(env, raising=False)
    monkeypatch.setattr(tuning, "_TUNING_CONFIG", {})
    return monkeypatch


def test_every_knob_has_its_default_first_and_distinct_envs():
    envs = [env for env, _ in tuning.KNOBS.values()]
    assert len(envs) == len(set(envs)) and all(e.startswith("MHC_") for e in envs)
    for env, cands in tuning.KNOBS.values():
        assert cands and len(cands) == len(set(cands)) and all(isinstance(c, int) for c in cands)


def test_every_knob_is_read_by_the_library():
    import pathlib

    csrc = pathlib.Path(__file__).resolve().parents[1] / "mhc-mlx_amd" / "csrc"
    text = "".join(p.read_text() for p in csrc.glob("*.hip"))
    for env in KNOB_ENVS:
        assert f'"{env}"' in text, env


def test_load_exports_knobs_and_later_files_win(tmp_path, clean_env):
    a, b = tmp_path / "a.json", tmp_path / "b.json"
    a.write_text(json.dumps({"residual_add_agg": {"MHC_RES_GRID": 8}, "sinkhorn_16": {"MHC_SK16_CPL": 2}}))
    b.write_text(json.dumps({"residual_add_agg": {"MHC_RES_GRID": 16}, "_device": "x"}))
    cfg = tuning.load([str(a), str(tmp_path / "missing.json"), str(b)])
    assert cfg["residual_add_agg"] == {"MHC_RES_GRID": 16}
    assert os.environ["MHC_RES_GRID"] == "16" and os.environ["MHC_SK16_CPL"] == "2"


def test_explicit_environment_wins(tmp_path, clean_env):
    clean_env.setenv("MHC_RES_GRID", "4")
    f = tmp_path / "t.json"
    f.write_text(json.dumps({"residual_add_agg": {"MHC_RES_GRID": 16}}))
    tuning.load([str(f)])
    assert os.environ["MHC_RES_GRID"] == "4"
    assert tuning.apply({"residual_add_agg": {"MHC_RES_GRID": 16}}, override=True) == {"MHC_RES_GRID": 16}
    assert os.environ["MHC_RES_GRID"] == "16"


def test_reference_format_entries_are_threadgroup_sizes(tmp_path, clean_env):
    """A file written by the reference's scripts/tune.py: {kernel: tpg}."""
    f = tmp_path / "mhc_tuning.json"
    f.write_text(json.dumps({"residual_add_agg": 512, "stream_mix_add": 128, "sinkhorn_128": 64}))
    tuning.load([str(f)])
    assert _get_tuned_tpg("stream_mix_add", 256) == 128
    assert _get_tuned_tpg("not_tuned", 256) == 256
    assert not any(env in os.environ for env in KNOB_ENVS)


def test_invalid_entries_apply_nothing(tmp_path, clean_env):
    f = tmp_path / "bad.json"
    f.write_text(json.dumps({"residual_add_agg": {"MHC_RES_GRID": 8}, "x": {"MHC_NOT_A_KNOB": 1}}))
    with pytest.warns(UserWarning, match="not applied"):
        tuning.load([str(f)])
    assert "MHC_RES_GRID" not in os.environ
    with pytest.raises(ValueError, match="integer"):
        tuning.apply({"sinkhorn_16": {"MHC_SK16_CPL": "4"}})
    g = tmp_path / "garbage.json"
    g.write_text("{not json")
    assert tuning.load([str(g)]) == {}


def test_tuner_needs_a_gpu():
    import torch

    from mhc_mlx_amd import tune

    if torch.cuda.is_available():
        pytest.skip("a GPU is present; covered by tests/test_gpu_tuning.py")
    with pytest.raises(RuntimeError, match="GPU"):
        tune.tune(scale=0.01)
