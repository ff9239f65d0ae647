"""The C-ABI library builds, loads and exports every entry point include/*.h declares."""
import re
from pathlib import Path

import rxmet_gru_abi  # noqa: F401  (registers the GRU signatures)
import rxmet_lstm_abi  # noqa: F401  (registers the LSTM signatures)
import rxmet_qc_abi  # noqa: F401  (registers the QcQuantizeOp signatures)
import rxmet_lib

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(rxmet_[a-z0-9_]+)\s*\(", text))
    return names


def test_headers_declare_entry_points():
    names = declared_symbols()
    assert "rxmet_qdq_forward" in names and "rxmet_last_error" in names


def test_library_exports_every_declared_symbol():
    lib = rxmet_lib.load()
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, f"librxmet.so lacks {missing}"


def test_python_signatures_cover_headers():
    assert declared_symbols() <= set(rxmet_lib.exported()), \
        sorted(declared_symbols() - set(rxmet_lib.exported()))


def test_host_only_calls_work_without_gpu():
    lib = rxmet_lib.load()
    assert lib.rxmet_abi_version() >= 1
    # [8192, 8192] per-channel on dim 0: 4096-element chunks (256 threads x four 16-byte vectors
    # of fp32); 8192 rows of two chunks are one workgroup each, one 16-byte partial per row.
    # Per-tensor: 16384 chunks, two per workgroup
    assert lib.rxmet_qdq_workspace_bytes(1, 8192, 8192) == 8192 * 16
    assert lib.rxmet_qdq_workspace_bytes(1, 1, 8192 * 8192) == 8192 * 16
    # 64 rows: too few for whole-row workgroups, two chunks per row
    assert lib.rxmet_qdq_workspace_bytes(1, 64, 8192) == 64 * 2 * 16
    # per-tensor below 2048 chunks: one chunk per workgroup
    assert lib.rxmet_qdq_workspace_bytes(1, 1, 4096 * 2047) == 2047 * 16


def test_noalloc_backward_rejects_layouts_beyond_its_scratch():
    """The size check of rxmet_qdq_backward_noalloc runs on the host before any device call:
    a layout whose partials exceed the 4 MiB scratch returns -22 with a message, no GPU needed."""
    import ctypes

    lib = rxmet_lib.load()
    buf = (ctypes.c_float * 4)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    n = 1 << 33  # per-tensor: 2^33 / 8192 partials (two 4096-element chunks each) of 16 bytes = 16 MiB
    need = lib.rxmet_qdq_workspace_bytes(1, 1, n)
    assert need > 4 << 20
    rc = lib.rxmet_qdq_backward_noalloc(p, p, p, p, p, 1, 1, n, p, p, -128, 127, 0, None)
    assert rc == -22
    msg = lib.rxmet_last_error().decode()
    assert "scratch" in msg and str(need) in msg, msg
