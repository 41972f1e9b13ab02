"""The C-ABI library loads, exports every symbol include/ declares, and reports
errors through LlaisysError (no compute calls: runs without a GPU)."""
import ctypes
import re
from pathlib import Path

import pytest

import llaisys_amd as L
from llaisys_amd.libllaisys import LIB_LLAISYS, LIB_PATH

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for h in (ROOT / "include").rglob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("#"))
        for m in re.finditer(r"__export\s+[^;(]*?\b(\w+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_headers_declare_the_reference_surface_plus_paged_ops():
    names = set(declared_symbols())
    reference = {  # include/llaisys/{tensor,runtime,ops}.h of the reference
        "tensorCreate", "tensorDestroy", "tensorGetData", "tensorGetNdim", "tensorGetShape", "tensorGetStrides",
        "tensorGetDataType", "tensorGetDeviceType", "tensorGetDeviceId", "tensorDebug", "tensorIsContiguous",
        "tensorLoad", "tensorView", "tensorPermute", "tensorSlice", "llaisysGetRuntimeAPI",
        "llaisysSetContextRuntime", "llaisysAdd", "llaisysArgmax", "llaisysEmbedding", "llaisysLinear",
        "llaisysRearrange", "llaisysRmsNorm", "llaisysROPE", "llaisysSelfAttention", "llaisysSwiGLU",
    }
    assert reference <= names
    assert {"llaisysPagedKVAppend", "llaisysPagedKVGather", "llaisysPagedAttention",
            "llaisysPagedAttentionVarlen"} <= names


@pytest.mark.parametrize("name", declared_symbols())
def test_library_exports_declared_symbol(name):
    lib = ctypes.CDLL(str(LIB_PATH))
    assert hasattr(lib, name), f"{name} declared in include/ but not exported"


@pytest.mark.parametrize("op", ["add", "argmax", "embedding", "rearrange", "swiglu"])
def test_model_ops_on_cpu_tensors_validate_arguments(op):
    # Host tensors run the CPU implementations; argument errors still fail
    # loudly (argmax needs an I64 index output, embedding an I64 index).
    t = L.Tensor((2,), dtype=L.DataType.F32)
    args = {"add": 3, "argmax": 3, "embedding": 3, "rearrange": 2, "swiglu": 3}[op]
    if op in ("argmax", "embedding"):
        with pytest.raises(L.LlaisysError):
            getattr(L.Ops, op)(*([t] * args))
    else:
        getattr(L.Ops, op)(*([t] * args))


def test_paged_ops_reject_bad_dtypes_and_shapes():
    pool = L.Tensor((4, 2, 16, 128), dtype=L.DataType.BF16)
    q = L.Tensor((2, 12, 128), dtype=L.DataType.BF16)
    out = L.Tensor((2, 12, 128), dtype=L.DataType.BF16)
    table = L.Tensor((2, 2), dtype=L.DataType.I32)
    ctx = L.Tensor((2,), dtype=L.DataType.I32)
    with pytest.raises(L.LlaisysError, match="q must be bf16"):
        L.Ops.paged_attention(out, L.Tensor((2, 12, 128), dtype=L.DataType.F32), pool, pool, table, ctx, 0.1)
    bad_pool = L.Tensor((4, 2, 8, 128), dtype=L.DataType.BF16)
    with pytest.raises(L.LlaisysError, match="pool must be"):
        L.Ops.paged_attention(out, q, bad_pool, bad_pool, table, ctx, 0.1)
    q13 = L.Tensor((2, 13, 128), dtype=L.DataType.BF16)
    with pytest.raises(L.LlaisysError, match="nh % nkvh"):
        L.Ops.paged_attention(L.Tensor((2, 13, 128), dtype=L.DataType.BF16), q13, pool, pool, table, ctx, 0.1)
    with pytest.raises(L.LlaisysError, match="one token per sequence"):
        kn = L.Tensor((3, 2, 128), dtype=L.DataType.BF16)
        L.Ops.paged_kv_append(pool, pool, kn, kn, table, ctx)


def test_self_attention_shape_checks():
    q = L.Tensor((3, 4, 8), dtype=L.DataType.F32)
    k = L.Tensor((2, 2, 8), dtype=L.DataType.F32)
    with pytest.raises(L.LlaisysError, match="total_len"):
        L.Ops.self_attention(L.Tensor((3, 4, 8), dtype=L.DataType.F32), q, k, k, 0.3)
    k3 = L.Tensor((5, 3, 8), dtype=L.DataType.F32)
    with pytest.raises(L.LlaisysError, match="multiple of nkvh"):
        L.Ops.self_attention(L.Tensor((3, 4, 8), dtype=L.DataType.F32), q, k3, k3, 0.3)


def test_last_error_is_cleared_after_read():
    buf = ctypes.create_string_buffer(256)
    assert LIB_LLAISYS.llaisysGetLastError(buf, 256) == 0


def test_one_hip_runtime_whatever_the_import_order():
    # Importing llaisys_amd before torch must not map a second libamdhip64.
    import subprocess
    import sys

    code = (
        "import os, llaisys_amd, torch\n"
        "maps = open(f'/proc/{os.getpid()}/maps').read().splitlines()\n"
        "hip = {l.split()[-1] for l in maps if 'amdhip64' in l and 'r-xp' in l}\n"
        "print(len(hip))\n"
    )
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, cwd=str(ROOT))
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "1"


def test_library_links_no_gemm_library():
    # The GEMMs are this project's own kernels: libllaisys.so needs no rocBLAS
    # or hipBLASLt (its dynamic section names the HIP runtime and libc++ only).
    import subprocess

    from llaisys_amd.libllaisys import LIB_PATH

    r = subprocess.run(["readelf", "-d", str(LIB_PATH)], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("readelf unavailable")
    needed = [l for l in r.stdout.splitlines() if "NEEDED" in l]
    assert needed and not any("blas" in l for l in needed), needed


def test_qwen2_create_rejects_cpu_and_non_bf16():
    from llaisys_amd.models import Qwen2, Qwen2Meta

    meta = Qwen2Meta(nlayer=1, hs=64, nh=2, nkvh=1, di=64, voc=32)
    with pytest.raises(L.LlaisysError, match="AMD"):
        Qwen2(meta=meta, device=L.DeviceType.CPU)
