"""CPU-side checks of the C ABI: the built library loads and exports every
entry point include/ax_hip_sampler.h declares (no GPU call is made)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    with open(os.path.join(ROOT, "include", "ax_hip_sampler.h")) as f:
        src = f.read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(axs_[a-z_]+)\s*\(", src)))


def test_header_declares_the_entry_points():
    fns = header_functions()
    for f in ("axs_context_create", "axs_context_destroy", "axs_sample_batch",
              "axs_argmax_batch", "axs_mtp_verify", "axs_last_error", "axs_abi_version"):
        assert f in fns


def test_library_exports_every_declared_symbol():
    from ax_sampler import _abi

    assert os.path.exists(_abi.LIB_PATH), "build first: __graft_entry__.build()"
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (axs_[a-z_]+)\b", out))
    missing = [f for f in header_functions() if f not in exported]
    assert not missing, missing
    assert set(_abi.EXPORTS) <= exported


def test_library_loads_without_touching_the_gpu():
    from ax_sampler import _abi

    L = ctypes.CDLL(_abi.LIB_PATH)
    L.axs_abi_version.restype = ctypes.c_int
    assert L.axs_abi_version() == 2
    L.axs_last_error.restype = ctypes.c_char_p
    assert L.axs_last_error() == b""


def test_struct_layouts_match_the_header():
    from ax_sampler import _abi
    from ax_sampler.params import PARAMS_DTYPE

    assert PARAMS_DTYPE.itemsize == 64
    assert ctypes.sizeof(_abi.BatchDesc) == 120
    assert ctypes.sizeof(_abi.Outputs) == 48
    assert ctypes.sizeof(_abi.MtpDesc) == 72
    assert ctypes.sizeof(_abi.MtpOutputs) == 32
    assert ctypes.sizeof(_abi.MtpOptions) == 48


def test_c_struct_sizes_from_the_compiler(tmp_path):
    src = tmp_path / "s.c"
    src.write_text(
        '#include "ax_hip_sampler.h"\n#include <stdio.h>\n#include <stddef.h>\n'
        "int main(){printf(\"%zu %zu %zu %zu %zu\\n\", sizeof(axs_sampling_params),"
        " sizeof(axs_batch_desc), sizeof(axs_outputs), sizeof(axs_mtp_desc),"
        " sizeof(axs_mtp_outputs)); printf(\"%zu\\n\", sizeof(axs_mtp_options)); return 0;}\n")
    exe = tmp_path / "s"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    sizes = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    assert sizes == ["64", "120", "48", "72", "32", "48"]


def test_error_handler_and_last_error_without_a_gpu():
    """A call refused before any HIP call (bad sizes) sets the thread's last
    error and calls the registered handler on this thread with the same
    message; unregistering stops the calls."""
    from ax_sampler import _abi

    L = ctypes.CDLL(_abi.LIB_PATH)
    L.axs_last_error.restype = ctypes.c_char_p
    L.axs_context_create.restype = ctypes.c_int
    L.axs_context_create.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]
    HANDLER = ctypes.CFUNCTYPE(None, ctypes.c_char_p, ctypes.c_void_p)
    seen = []
    h = HANDLER(lambda msg, data: seen.append((msg, data)))
    L.axs_set_error_handler.argtypes = [HANDLER, ctypes.c_void_p]
    L.axs_set_error_handler(h, ctypes.c_void_p(1234))
    out = ctypes.c_void_p()
    assert L.axs_context_create(0, 0, 10, ctypes.byref(out)) == 1  # AXS_E_INVALID
    assert out.value is None
    assert L.axs_last_error() == b"max_batch and max_vocab must be >= 1"
    assert seen == [(b"max_batch and max_vocab must be >= 1", 1234)]
    L.axs_set_error_handler(HANDLER(), None)
    assert L.axs_context_create(0, 10, -1, ctypes.byref(out)) == 1
    assert len(seen) == 1


def test_new_entry_points_refuse_bad_arguments_without_a_gpu():
    """axs_lm_head and axs_mtp_draft validate their arguments before any HIP
    call: a NULL context or a shape they cannot take is AXS_E_INVALID with a
    message, on a machine without a GPU."""
    from ax_sampler import _abi

    L = ctypes.CDLL(_abi.LIB_PATH)
    L.axs_last_error.restype = ctypes.c_char_p
    vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    L.axs_lm_head.restype = i32
    L.axs_lm_head.argtypes = [vp, vp, i64, vp, i64, i32, i32, i32, f32, f32, vp, i64, vp, vp]
    L.axs_mtp_draft.restype = i32
    L.axs_mtp_draft.argtypes = [vp, vp, i32, i32, i32, i64, vp, i32, vp, vp, vp, vp]
    p = ctypes.c_void_p(16)  # never dereferenced: refused first
    assert L.axs_lm_head(None, p, 64, p, 64, 1, 64, 10, 1.0, 0.0, p, 10, p, None) == 1
    assert b"non-NULL" in L.axs_last_error()
    assert L.axs_mtp_draft(None, p, 0, 1, 10, 10, p, 0, None, p, p, None) == 1
    assert b"non-NULL" in L.axs_last_error()
