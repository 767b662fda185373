"""The C ABI library loads and exports every symbol include/llamatov_hip.h declares;
argument validation and the host-only helpers work without a GPU."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from llamatov_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    txt = (ROOT / "include" / "llamatov_hip.h").read_text()
    return sorted(set(re.findall(r"^LT_API\s+(?:int|size_t)\s+(lt_\w+)\s*\(", txt, flags=re.M)))


def test_header_and_binding_agree():
    assert sorted(_lib.exported_symbols()) == declared_symbols()


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_library_hides_internal_symbols():
    # only the C ABI is visible; kernels and helpers stay internal
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    names = {l.split()[-1] for l in out.splitlines() if l.strip()}
    lt = {n for n in names if n.startswith("lt_")}
    assert lt == set(declared_symbols())


def test_validation_errors_without_gpu():
    lib = _lib.load()
    P = ctypes.c_void_p
    assert lib.lt_quant_q8(None, P(0), P(0), P(0), 32) == -1
    assert "null" in _lib.last_error()
    assert lib.lt_q8_gemv(None, P(0), P(0), P(0), P(0), P(0), 8, 33) == -1
    assert lib.lt_argmax(None, P(0), 0, P(0), P(0), 0) == -1
    assert lib.lt_graph_launch(None, None) == -1
    with pytest.raises(_lib.LtError):
        _lib.call("lt_rmsnorm", None, P(0), P(0), P(0), 1, 896, ctypes.c_float(1e-6))


def test_workspace_sizes():
    lib = _lib.load()
    assert lib.lt_attn_workspace_size(1, 32, 128, 1) == 0
    assert lib.lt_attn_workspace_size(8, 32, 128, 64) >= 8 * 32 * 64 * 130 * 4
    assert lib.lt_argmax_workspace_size() >= 256 * 8


def test_rope_freqs_host_helper_matches_oracle(oracle):
    for hd, theta in ((64, 1e6), (128, 5e5), (32, 1e4)):
        f = np.empty(hd // 2, np.float32)
        assert _lib.load().lt_rope_freqs(hd, ctypes.c_float(theta), f.ctypes.data_as(ctypes.c_void_p)) == 0
        assert np.array_equal(f, oracle.rope_freqs(hd, theta))
