"""The rates calibration on the device: every key of the shipped file
measured, each inside what MI355X can do."""
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def test_calibration_measures_every_key(target):
    from tempest_hip import calibrate
    announce("calibrate")
    r = calibrate.calibrate(target)
    assert r["timing basis"] == calibrate.TIMING_BASIS
    assert 7e12 < r["device bandwidth"] < 9e12 and r["device blocks"] == 256
    assert 0 < r["floor memory latency"] < 2e-5 and 2e12 < r["floor memory bandwidth"] <= r["device bandwidth"]
    assert 5e14 < r["HIP BFloat16 rate"] < 2.5e15
    for name, _ in calibrate.APPLIED:
        assert 0.0 <= r[f"applied streamed any {name}"] < 1e-10, name
    assert r["applied streamed any sin"] > r["applied streamed any +"]
