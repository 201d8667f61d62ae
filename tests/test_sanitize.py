"""AddressSanitizer and UndefinedBehaviorSanitizer runs on the CPU (no GPU).

- The C oracle (``oracle/cpu_ref.c``) linked with ``tests/sanitize/oracle_probe.c``:
  every exported function on exact-size buffers, empty inputs included.
- The library's host code (every source under ``keep_amd/csrc``, host side
  instrumented) linked with ``tests/sanitize/abi_probe.cpp``: every C-ABI entry
  point called with all-zero / all-null, -1 / NaN and huge arguments must
  return KEEP_OK or KEEP_EINVAL, with no out-of-bounds access and no undefined
  behaviour in its checks (a size product that overflows int64, say), then the
  host-only entry points on valid buffers.

The build (``tests/sanitize/build.sh``, about two minutes) is cached under
``keep_amd/_build/san`` and redone when a source changes."""

import hashlib
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
OUT = ROOT / "keep_amd" / "_build" / "san"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _sources():
    return [*sorted((ROOT / "keep_amd" / "csrc").iterdir()), *sorted((ROOT / "tests" / "sanitize").iterdir()),
            ROOT / "oracle" / "cpu_ref.c", ROOT / "include" / "keep_amd.h"]


@pytest.fixture(scope="module")
def san() -> Path:
    if not Path(HIPCC).exists() or shutil.which("gcc") is None:
        pytest.skip("hipcc and gcc are needed for the sanitizer builds")
    h = hashlib.sha256()
    for p in _sources():
        if p.is_file():
            h.update(p.name.encode())
            h.update(p.read_bytes())
    digest = h.hexdigest()
    stamp = OUT / "sources.sha256"
    fresh = stamp.exists() and stamp.read_text() == digest
    if not (fresh and (OUT / "abi_probe").exists() and (OUT / "oracle_probe").exists()):
        stamp.unlink(missing_ok=True)
        res = subprocess.run(["bash", str(ROOT / "tests" / "sanitize" / "build.sh"), str(OUT)], capture_output=True,
                             text=True, timeout=1200)
        assert res.returncode == 0, res.stderr[-4000:]
        stamp.write_text(digest)
    return OUT


def _run(exe: Path, **env) -> subprocess.CompletedProcess:
    return subprocess.run([str(exe)], capture_output=True, text=True, timeout=300,
                          env={**os.environ, "OMP_NUM_THREADS": "2", **env})


def test_c_oracle_under_asan_and_ubsan(san):
    r = _run(san / "oracle_probe")
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stderr[-4000:]
    assert "runtime error" not in r.stderr


def test_abi_argument_checks_under_asan_and_ubsan(san):
    # the HIP runtime keeps allocations until exit: leak reports would be its own
    r = _run(san / "abi_probe", ASAN_OPTIONS="detect_leaks=0:verify_asan_link_order=0")
    assert r.returncode == 0 and "ok: 0 failures" in r.stdout, (r.stdout[-2000:], r.stderr[-4000:])
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr
