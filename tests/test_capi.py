"""The C ABI library (CPU): it loads, exports every entry point that
include/tierkv_hip.h declares, and rejects bad arguments before any launch;
the Python wrappers raise the reference's exception types."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from paged_tierkv_amd import _lib
from paged_tierkv_amd.tierkv_hip import tierkv_decode_attention

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tierkv_hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"TIERKV_API\s+[\w\s\*]+?\b(tierkv_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = _declared()
    assert len(names) >= 19
    lib = _lib.lib()
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (tierkv_\w+)", out))
    assert exported == set(names), exported ^ set(names)


def test_python_constants_match_the_header():
    defines = {m.group(1): int(m.group(2), 0)
               for m in re.finditer(r"#define\s+(TIERKV_\w+)\s+(0x[0-9a-fA-F]+|\d+)", open(HEADER).read())}
    pairs = {"TIERKV_OK": _lib.TIERKV_OK, "TIERKV_ERR_INVALID": _lib.TIERKV_ERR_INVALID,
             "TIERKV_ERR_UNSUPPORTED": _lib.TIERKV_ERR_UNSUPPORTED, "TIERKV_ERR_HIP": _lib.TIERKV_ERR_HIP,
             "TIERKV_ERR_WORKSPACE": _lib.TIERKV_ERR_WORKSPACE, "TIERKV_ERR_STATE": _lib.TIERKV_ERR_STATE,
             "TIERKV_DTYPE_F16": _lib.DTYPE_F16, "TIERKV_DTYPE_BF16": _lib.DTYPE_BF16,
             "TIERKV_WARM_REF_U8": _lib.WARM_REF_U8, "TIERKV_WARM_ABSMAX_I8": _lib.WARM_ABSMAX_I8,
             "TIERKV_COLD_ZERO_LOGIT": _lib.COLD_ZERO_LOGIT, "TIERKV_COLD_MASKED": _lib.COLD_MASKED,
             "TIERKV_DECODE_DETERMINISTIC": _lib.DECODE_DETERMINISTIC}
    for name, value in pairs.items():
        assert defines[name] == value, name


def test_decode_workspace_bytes_ignore_the_deterministic_flag():
    lib = _lib.lib()
    for splits in (0, 1, 3, 8):
        a = lib.tierkv_decode_workspace_bytes(4, 32, 8, 2048, 16, 128, 1, splits)
        b = lib.tierkv_decode_workspace_bytes(4, 32, 8, 2048, 16, 128, 1, splits | _lib.DECODE_DETERMINISTIC)
        assert a == b > 0


def test_abi_version_and_errors_without_gpu():
    lib = _lib.lib()
    assert lib.tierkv_abi_version() == _lib.ABI_VERSION
    rc = lib.tierkv_decode_attention(
        None, 0, None, None,            # query, dtype, out, score_sums
        None, None, None, 0, None, 0,   # table, states, lengths, stride, seq_num_blocks, num_blocks
        None, None, 0, None, None, 0,   # hot pools + slots, warm pools + slots
        None, None, None, None, 0, 0,   # scales / zeros, warm format, cold mode
        0, 0, 0, 0, 0,                  # batch, heads, kv heads, block size, head dim
        ctypes.c_float(1.0), 0, None, 0, None)
    assert rc == _lib.TIERKV_ERR_INVALID
    assert "null" in _lib.last_error()
    assert lib.tierkv_decode_workspace_bytes(0, 1, 1, 1, 16, 64, 0, 0) < 0
    assert lib.tierkv_decode_workspace_bytes(32, 32, 8, 256, 16, 128, 1, 0) > 0
    assert lib.tierkv_tier_labels(None, None, None, 4, 1, 4, 2, 1, 7, 1, None) == _lib.TIERKV_ERR_INVALID
    assert lib.tierkv_block_mass_from_probs(None, None, None, 1, 1, 16, 16, None) == _lib.TIERKV_ERR_INVALID
    assert lib.tierkv_decode_noalloc_error_word(1, None) == _lib.TIERKV_ERR_INVALID


def test_decode_wrapper_contract_on_cpu_tensors():
    q = torch.zeros((1, 8, 1, 64), dtype=torch.float16)
    table = torch.zeros(4, dtype=torch.int32)
    pool = torch.zeros((2, 4, 16, 64), dtype=torch.float16)
    wpool = torch.zeros((2, 4, 16, 64), dtype=torch.uint8)
    meta = torch.ones((2, 4, 16, 1), dtype=torch.float16)
    args = [table, table, table, pool, pool, wpool, wpool, meta, meta, meta, meta]
    with pytest.raises(ValueError, match="shape"):
        tierkv_decode_attention(q[0], *args, num_blocks=2, num_key_value_groups=2, scaling=0.125)
    with pytest.raises(ValueError, match="batch size 1"):
        tierkv_decode_attention(q.repeat(2, 1, 1, 1), *args, num_blocks=2, num_key_value_groups=2, scaling=0.125)
    with pytest.raises(ValueError, match="query_len"):
        tierkv_decode_attention(q.repeat(1, 1, 2, 1), *args, num_blocks=2, num_key_value_groups=2, scaling=0.125)
    with pytest.raises(ValueError, match="GPU"):
        tierkv_decode_attention(q, *args, num_blocks=2, num_key_value_groups=2, scaling=0.125)


def test_missing_library_raises_runtime_error(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libtierkv_hip.so")
    with pytest.raises(RuntimeError, match="not built"):
        _lib.lib()


def test_decode_step_struct_layout_matches_header(tmp_path):
    """Every TierkvDecodeStep field sits where the ctypes mirror puts it:
    offsets printed by a C program compiled against the header."""
    fields = [name for name, _ in _lib.DecodeStep._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "tierkv_hip.h"\nint main(void) {\n'
                   '  printf("%zu\\n", sizeof(TierkvDecodeStep));\n'
                   + "".join(f'  printf("%zu\\n", offsetof(TierkvDecodeStep, {f}));\n' for f in fields)
                   + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got[0] == ctypes.sizeof(_lib.DecodeStep) == _lib.lib().tierkv_decode_step_size()
    assert got[1:] == [getattr(_lib.DecodeStep, f).offset for f in fields]


def test_decode_step_rejects_bad_counts_without_gpu():
    lib = _lib.lib()
    assert lib.tierkv_decode_step(None, None) == _lib.TIERKV_ERR_INVALID
    assert "null" in _lib.last_error()
    st = _lib.DecodeStep()
    st.n_jobs = 5
    assert lib.tierkv_decode_step(ctypes.byref(st), None) == _lib.TIERKV_ERR_INVALID
    assert "write jobs" in _lib.last_error()
    st.n_jobs, st.n_pairs = 0, 17
    assert lib.tierkv_decode_step(ctypes.byref(st), None) == _lib.TIERKV_ERR_INVALID
    assert "table writes" in _lib.last_error()
    st.n_jobs, st.n_pairs = 1, 0   # a write job with no source or pool pointers
    assert lib.tierkv_decode_step(ctypes.byref(st), None) == _lib.TIERKV_ERR_INVALID
    assert "null" in _lib.last_error()
