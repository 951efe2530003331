"""The probe's correctness gates (astc_kv.probe) on the CPU, against the
reference's refusal controls (scripts/verify_metal_v4.py:24-45): the same
fixture with one offline-decoded value moved by +1000, made NaN, or with the
offline decode missing must be refused (status correctness_failed, no raw
samples); the fixture itself passes. The GPU results the gates judge are
stood in for by the product CPU decoder (libakv_astc) and the fp32 NumPy
attention of astc_kv.codec; tests/test_gpu_probe.py runs the real thing."""
import copy

import numpy as np
import pytest

from astc_kv import codec, probe


@pytest.fixture(scope="module")
def fixture(golden):
    return probe.load_fixture(golden / "t384" / "manifest.json")


def _standins(fx):
    v = fx["atlas"].restored().astype(np.float32)          # [1, Hkv, T, D]
    out, _ = codec.attention(fx["q"][0][:, None], fx["k"][0].astype(np.float32), v[0], [fx["k"].shape[2] - 1])
    out16, _ = codec.attention(fx["q"][0][:, None], fx["k"][0].astype(np.float32),
                               v[0].astype(np.float16).astype(np.float32), [fx["k"].shape[2] - 1])
    return v, out[:, 0][None], out16[:, 0][None]


def test_fixture_passes(fixture):
    v, out, out16 = _standins(fixture)
    passed, c = probe.gates(fixture, v, out, out16)
    assert passed, c
    assert c["v_decode_gate"]["bit_exact"] and c["astc_decode_attention"]["passed_rtol_l2_1e_4"]


@pytest.mark.parametrize("control", ["wrong_decode", "nonfinite_decode", "missing_decode", "wrong_output"])
def test_controls_are_refused(fixture, control):
    fx = copy.copy(fixture)
    v, out, out16 = _standins(fx)
    if control == "missing_decode":
        fx["v_decoded"] = None
    elif control == "wrong_output":
        out = out + np.float32(1e-2)
    else:
        vd = fx["v_decoded"].copy()
        flat = vd.reshape(-1)
        flat[0] = np.nan if control == "nonfinite_decode" else flat[0] + 1000
        fx["v_decoded"] = vd
    passed, c = probe.gates(fx, v, out, out16)
    assert not passed
    rec = probe.refusal(c)
    assert rec["status"] == "correctness_failed" and rec["raw_samples"] == []
    if control == "missing_decode":
        assert c["v_decode_gate"]["reason"] == "Missing offline decode reference"
    elif control == "wrong_output":
        assert not c["astc_decode_attention"]["passed_rtol_l2_1e_4"]
    else:
        assert not c["v_decode_gate"]["passed"]


def test_unsupported_fixture(golden):
    with pytest.raises(probe.UnsupportedFixture):
        probe.load_fixture(golden / "kv_page6" / "manifest.json")


def test_fp64_reference_matches_codec_attention(fixture):
    v, out, _ = _standins(fixture)
    ref = probe.attention_fp64(fixture["q"][0], fixture["k"][0], v[0])
    np.testing.assert_allclose(out[0], ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("tokens", [391, 2048, 8192])
def test_repeated_fixture(fixture, tokens):
    """A fixture repeated to T keys (the reference's traffic controls,
    scripts/make_traffic_fixture.py:12-49): block rows cover T rounded up to
    whole pages, the decoded atlas is the offline decode repeated token by
    token, and the gates still pass on it."""
    fx = probe.repeat_tokens(fixture, tokens)
    a = fx["atlas"]
    assert a.tokens == tokens and fx["k"].shape[2] == tokens and fx["v_decoded"].shape[2] == tokens
    assert a.rows == -(-tokens // a.page_tokens) * a.page_tokens // a.block_y
    r = np.arange(a.rows) % fixture["atlas"].rows
    assert np.array_equal(a.blocks, fixture["atlas"].blocks[:, :, r])
    v = a.restored().astype(np.float32)
    assert np.array_equal(v.view(np.uint32), fx["v_decoded"].view(np.uint32))
    if tokens <= 2048:
        v, out, out16 = _standins(fx)
        passed, c = probe.gates(fx, v, out, out16)
        assert passed, c


def test_repeated_fixture_bounds(fixture):
    for bad in (0, 8193):
        with pytest.raises(ValueError):
            probe.repeat_tokens(fixture, bad)
