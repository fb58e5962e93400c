"""The C ABI: the built library loads and exports every symbol the header declares.

No compute call is made here (no GPU in the CPU suite)."""
import ctypes
import subprocess

from decisive_amd import rocm


def test_header_declares_entry_points():
    syms = rocm.header_symbols()
    for name in ("dz_init", "dz_weight_upload", "dz_linear", "dz_i8_gemm", "dz_tune", "dz_encoder_forward"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    lib = rocm.load()
    missing = [s for s in rocm.header_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", str(rocm.LIB_PATH)], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(rocm.header_symbols()) <= exported


def test_bindings_cover_the_header():
    assert set(rocm.header_symbols()) == set(rocm._SIGNATURES)


def test_status_names_match_reference_codes():
    lib = rocm.load()
    for code, name in rocm.STATUS_NAMES.items():
        assert lib.dz_status_name(code).decode() == name
    assert lib.dz_status_name(999).decode() == "UNKNOWN"


def test_init_without_gpu_reports_gpu_unavailable():
    import torch
    if torch.cuda.is_available():
        return
    h = ctypes.c_void_p()
    rc = rocm.load().dz_init(0, ctypes.byref(h))
    assert rocm.STATUS_NAMES[rc] in ("GPU_UNAVAILABLE", "MISSING_GPU_FEATURE")
    assert h.value is None
