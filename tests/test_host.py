"""The C++ host layer (decisive_amd/host): the reference's inference API
restated over the C ABI, run as compiled test programs."""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HOST = ROOT / "decisive_amd" / "host"
BUILD = HOST / "build"


def _program(name: str) -> Path:
    """The test program, rebuilt by make when a source or header changed."""
    exe = BUILD / name
    subprocess.run(["make", "-s", "-C", str(HOST), str(exe)], check=True)
    return exe


def _run(exe: Path, timeout: int):
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    print(r.stderr)
    return r


def test_model_cache_parameters_and_embedding_cache_on_cpu():
    """Ports of src/inference/tests.rs:57-141 plus EmbeddingCache
    (browser/pplx.rs:45-138) and error-code mapping (mod.rs:56-78)."""
    r = _run(_program("test_inference"), 60)
    assert r.returncode == 0, r.stderr
    assert "0 failed check(s)" in r.stdout


@pytest.mark.gpu
def test_rocm_backend_behind_model():
    """Model<Rocm> on the GPU: predictions equal the direct encoder forward bit
    for bit, cache reuse, splitting by maxSequenceTokens, failure clearing."""
    r = _run(_program("test_rocm_backend"), 120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failed check(s)" in r.stdout
