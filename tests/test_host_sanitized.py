"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer,
on the CPU: a check build (sanitizers on the host side only) runs the floor's
device-free tests (validation, planning, source writing, hiprtc compiles and
the code-object store) in a child process; any sanitizer report fails."""
import importlib.util
import os
import pathlib
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent.parent


def _build_module():
    spec = importlib.util.spec_from_file_location("tempest_hip_build", ROOT / "tempest.jl_amd" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_floor_host_code_is_clean_under_asan_and_ubsan(tmp_path):
    b = _build_module()
    lib = b.build_sanitized(tmp_path / "asan")
    env = dict(os.environ)
    env.update({
        "TEMPEST_HIP_LIBRARY": str(lib),
        "LD_PRELOAD": " ".join(p for p in (str(b.sanitizer_runtime()), env.get("LD_PRELOAD", "")) if p),
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
        "TEMPEST_HIP_CACHE": str(tmp_path / "store"),
    })
    p = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
                        str(ROOT / "tests" / "test_oracle_floor.py"), str(ROOT / "tests" / "test_floor_store.py")],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = p.stdout + p.stderr
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-6000:]
    assert p.returncode == 0, out[-6000:]
    assert " passed" in out
