"""The probe CLI (astc_kv.probe.main, run in this process) on the GPU: the
reference fixtures pass their gates and are timed; the reference's refusal
controls (scripts/verify_metal_v4.py:24-45: one offline-decoded value +1000,
one NaN, the offline decode missing), derived from the same fixture the way
that script derives them, are refused with status correctness_failed, no raw
samples and exit status 1, before any timing."""
import json
import shutil

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _control(golden, tmp_path, name):
    d = tmp_path / name
    shutil.copytree(golden / "t384", d)
    m = json.loads((d / "manifest.json").read_text())
    if name == "missing_decode":
        del m["v_decoded_file"]
    elif name in ("wrong_decode", "nonfinite_decode"):
        values = np.fromfile(d / m["v_decoded_file"], "<f4")
        values[0] = np.nan if name == "nonfinite_decode" else values[0] + 1000
        values.tofile(d / m["v_decoded_file"])
    (d / "manifest.json").write_text(json.dumps(m, indent=2) + "\n")
    return d / "manifest.json"


@pytest.mark.parametrize("name", ["t384", "t391"])
@pytest.mark.parametrize("tile", [13, 256])
def test_fixtures_pass_and_are_timed(golden, capsys, name, tile):
    from astc_kv import probe
    rc = probe.main([str(golden / name / "manifest.json"), "--tile", str(tile), "--rounds", "2", "--iterations", "3"])
    rec = json.loads(capsys.readouterr().out)
    assert rc == 0 and rec["status"] == "ok" and len(rec["raw_samples"]) == 2
    assert rec["correctness"]["v_decode_gate"]["bit_exact"]
    assert rec["tile_tokens"] == tile


@pytest.mark.parametrize("name", ["wrong_decode", "nonfinite_decode", "missing_decode"])
def test_controls_are_refused(golden, tmp_path, capsys, name):
    from astc_kv import probe
    rc = probe.main([str(_control(golden, tmp_path, name)), "--tile", "13", "--rounds", "2", "--iterations", "3"])
    out = capsys.readouterr()
    rec = json.loads(out.out)
    assert rc == 1 and rec["status"] == "correctness_failed" and rec["raw_samples"] == []
    assert "no timing result is published" in out.err
