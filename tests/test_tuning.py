"""The tuning file (mhc_mlx/metal.py:21-36, scripts/tune.py): loading, precedence and the
reference's integer entries (CPU)."""

import json
import os
import subprocess
import sys

import pytest

from mhc_mlx_amd import _lib, tuning
from mhc_mlx_amd.metal import _get_tuned_tpg

KNOB_ENVS = sorted({env for env, _ in tuning.KNOBS.values()})

pytestmark = pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="libmhc_hip.so not built")


@pytest.fixture
def clean_env(monkeypatch, knobs):
    """No knob in the environment or the library's table; the table is restored afterwards."""
    for env in KNOB_ENVS:
        monkeypatch.delenv(env, raising=False)
    for name in _lib.knob_names():
        knobs(name, None)
    monkeypatch.setattr(tuning, "_TUNING_CONFIG", {})
    return monkeypatch


def test_every_knob_has_its_default_first_and_distinct_envs():
    envs = [env for env, _ in tuning.KNOBS.values()]
    assert len(envs) == len(set(envs)) and all(e.startswith("MHC_") for e in envs)
    for env, cands in tuning.KNOBS.values():
        assert cands and len(cands) == len(set(cands)) and all(isinstance(c, int) for c in cands)


def test_every_knob_is_in_the_library_table():
    names = _lib.knob_names()
    assert len(names) == len(set(names)) and all(n.startswith("MHC_") for n in names)
    assert set(KNOB_ENVS) <= set(names), set(KNOB_ENVS) - set(names)


def test_knob_table_set_get_unset(clean_env):
    assert _lib.get_knob("MHC_BWD_GRID") is None
    _lib.set_knob("MHC_BWD_GRID", 12)
    assert _lib.get_knob("MHC_BWD_GRID") == 12
    _lib.set_knob("MHC_BWD_GRID", None)
    assert _lib.get_knob("MHC_BWD_GRID") is None
    with pytest.raises(ValueError, match="unknown knob"):
        _lib.set_knob("MHC_NOT_A_KNOB", 1)
    with pytest.raises(ValueError, match="unknown knob"):
        _lib.get_knob("MHC_NOT_A_KNOB")
    with pytest.raises(ValueError, match="integer"):
        _lib.set_knob("MHC_BWD_GRID", "3")
    assert "MHC_BWD_GRID" not in os.environ


def test_knobs_start_from_the_environment_at_load():
    """The library reads each knob's environment variable once, when it is loaded."""
    code = ("from mhc_mlx_amd import _lib; import os; print(_lib.get_knob('MHC_RES_GRID'), "
            "_lib.get_knob('MHC_SK16_CPL')); os.environ['MHC_SK16_CPL'] = '2'; print(_lib.get_knob('MHC_SK16_CPL'))")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = {k: v for k, v in os.environ.items() if not k.startswith("MHC_")}
    env.update(MHC_RES_GRID="7", PYTHONPATH=os.path.join(root, "mhc-mlx_amd"))
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300,
                         cwd=root)
    assert out.returncode == 0, out.stderr
    assert out.stdout.split() == ["7", "None", "None"]


def test_load_exports_knobs_and_later_files_win(tmp_path, clean_env):
    a, b = tmp_path / "a.json", tmp_path / "b.json"
    a.write_text(json.dumps({"residual_add_agg": {"MHC_RES_GRID": 8}, "sinkhorn_16": {"MHC_SK16_CPL": 2}}))
    b.write_text(json.dumps({"residual_add_agg": {"MHC_RES_GRID": 16}, "_device": "x"}))
    cfg = tuning.load([str(a), str(tmp_path / "missing.json"), str(b)])
    assert cfg["residual_add_agg"] == {"MHC_RES_GRID": 16}
    assert _lib.get_knob("MHC_RES_GRID") == 16 and _lib.get_knob("MHC_SK16_CPL") == 2
    assert "MHC_RES_GRID" not in os.environ  # the environment is never written


def test_explicit_environment_wins(tmp_path, clean_env):
    clean_env.setenv("MHC_RES_GRID", "4")
    f = tmp_path / "t.json"
    f.write_text(json.dumps({"residual_add_agg": {"MHC_RES_GRID": 16}}))
    tuning.load([str(f)])
    assert _lib.get_knob("MHC_RES_GRID") is None  # the environment's value is the library's (read at load)
    assert tuning.apply({"residual_add_agg": {"MHC_RES_GRID": 16}}, override=True) == {"MHC_RES_GRID": 16}
    assert _lib.get_knob("MHC_RES_GRID") == 16 and os.environ["MHC_RES_GRID"] == "4"


def test_reference_format_entries_are_threadgroup_sizes(tmp_path, clean_env):
    """A file written by the reference's scripts/tune.py: {kernel: tpg}."""
    f = tmp_path / "mhc_tuning.json"
    f.write_text(json.dumps({"residual_add_agg": 512, "stream_mix_add": 128, "sinkhorn_128": 64}))
    tuning.load([str(f)])
    assert _get_tuned_tpg("stream_mix_add", 256) == 128
    assert _get_tuned_tpg("not_tuned", 256) == 256
    assert all(_lib.get_knob(env) is None for env in KNOB_ENVS)


def test_invalid_entries_apply_nothing(tmp_path, clean_env):
    f = tmp_path / "bad.json"
    f.write_text(json.dumps({"residual_add_agg": {"MHC_RES_GRID": 8}, "x": {"MHC_NOT_A_KNOB": 1}}))
    with pytest.warns(UserWarning, match="not applied"):
        tuning.load([str(f)])
    assert _lib.get_knob("MHC_RES_GRID") is None
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
