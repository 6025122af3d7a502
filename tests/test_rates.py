"""The shipped MI355X rates file (tempest_hip.calibrate, measured on the
device): the reference's format and keys, and values inside what the device
can do (HBM 8 TB/s, bf16 2.5 PFLOP/s dense)."""
import pathlib

from tempest_hip import calibrate

RATES = pathlib.Path(__file__).resolve().parent.parent / "tempest.jl_amd" / "rates" / "AMD_Instinct_MI355X.cold.rates.tsv"


def test_rates_file_has_the_reference_keys_and_sane_values():
    r = calibrate.read(RATES)
    assert r["timing basis"] == calibrate.TIMING_BASIS  # the reference's record.jl:182 definition
    assert 7e12 < r["device bandwidth"] < 9e12 and r["device blocks"] == 256 and r["device cache"] > 2.56e8
    assert 1e-7 < r["floor memory latency"] < 2e-5
    assert 2e12 < r["floor memory bandwidth"] <= r["device bandwidth"]
    assert 5e14 < r["HIP BFloat16 rate"] < 2.5e15 and r["HIP BFloat16 split"] == r["HIP BFloat16 rate"]
    for name, _ in calibrate.APPLIED:
        v = r[f"applied streamed any {name}"]
        assert 0.0 <= v < 1e-10, name
    # Transcendentals cost more than a multiply in a streamed fold.
    assert r["applied streamed any exp"] > r["applied streamed any *"]
