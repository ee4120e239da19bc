"""The C ABI of libdgen_hip.so on a host without a GPU: the library loads,
exports every entry point include/dgen_hip.h declares, and reports errors
through status codes and dgen_hip_last_error() instead of aborting."""
import ctypes
import os
import re
import subprocess

import numpy as np

import dgen_hip
from dgen_hip import runtime as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dgen_hip.h")
PROCESS_HEADER = os.path.join(ROOT, "include", "dgen_process_v1.h")


def declared(header=HEADER, prefix="dgen_hip_"):
    text = open(header).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(" + prefix + r"\w+)\s*\(", text, re.M)))


def test_header_declares_the_runtime_interface():
    names = declared()
    for n in ("dgen_hip_create", "dgen_hip_configure", "dgen_hip_run", "dgen_hip_host_memory", "dgen_hip_profile",
              "dgen_hip_last_error", "dgen_hip_destroy"):
        assert n in names
    assert set(names) == set(R.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(R.LIB_PATH)
    missing = [n for n in declared() + declared(PROCESS_HEADER, "dgen_") if not hasattr(lib, n)]
    assert not missing, missing


def test_process_header_declares_the_reference_exports():
    # dgen_runtime.h:283-291: exactly these two symbols
    assert declared(PROCESS_HEADER, "dgen_") == sorted(R.PROCESS_V1_SYMBOLS)


def test_process_exports_unbound_return_silence_and_a_message():
    L = dgen_hip.load_library()
    assert L.dgen_hip_process_memory_size() == 0
    out = np.ones((1, 32), np.float32)
    state = np.zeros(1024, np.float32)
    # nothing bound: the call returns (void), leaves the state block alone
    got = R.process_v1([], 1, 32, state)
    assert b"no schedule bound" in L.dgen_hip_last_error()
    assert not np.any(state) and got.shape == out.shape
    L.dgen_set_param_value_v1(3, 1.0)  # the reference C backend's no-op
    assert L.dgen_hip_process_bind(None, 0, 16) == 0  # unbinding is always allowed


def test_a_c_host_resolves_the_process_exports_by_name(tmp_path):
    exe = tmp_path / "process_host"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "process_host.c"), "-o", str(exe), "-ldl"], check=True)
    r = subprocess.run([str(exe), R.LIB_PATH], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert "no schedule bound" in r.stdout


def test_kernel_class_ids_match_header():
    text = open(HEADER).read()
    ids = dict((k, int(v)) for k, v in re.findall(r"DGEN_HIP_K_(\w+)\s*=\s*(\d+)", text))
    for name, v in ids.items():
        assert getattr(R, "K_" + name) == v, name


def test_errors_are_status_codes_not_aborts():
    L = dgen_hip.load_library()
    assert L.dgen_hip_abi_version() == 2
    rc = L.dgen_hip_run(None, 16)
    assert rc == -3 and b"not configured" in L.dgen_hip_last_error()
    assert L.dgen_hip_set_outputs(None, 0, 4) == -3
    n = ctypes.c_uint64(7)
    assert not L.dgen_hip_host_outputs(None, ctypes.byref(n)) and n.value == 0
    assert L.dgen_hip_set_sample_rate(None, 44100.0) == -1
    rc = L.dgen_hip_configure(None, None, 0, 0, 0)
    assert rc == -1 and L.dgen_hip_last_error()
    n = ctypes.c_int(-1)
    rc = L.dgen_hip_device_count(ctypes.byref(n))
    assert (rc == 0 and n.value >= 0) or (rc == -2 and n.value == 0)
    if rc != 0 or n.value == 0:
        ctx = ctypes.c_void_p()
        assert L.dgen_hip_create(0, ctypes.byref(ctx)) < 0 and ctx.value is None
        assert dgen_hip.device_count() == 0
