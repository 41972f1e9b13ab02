"""The xmake build (xmake.lua + xmake/hip.lua, the reference's build hook
pattern of xmake.lua:10-19) and llaisys_amd/build.py compile the same sources
with the same hipcc flags. xmake itself is not installed in this image, so the
check reads the Lua files."""
import re
from pathlib import Path

from llaisys_amd import build as B

ROOT = Path(__file__).resolve().parents[1]


def _lua_flags():
    text = (ROOT / "xmake" / "hip.lua").read_text()
    block = text.split("-- HIP_FLAGS_BEGIN", 1)[1].split("-- HIP_FLAGS_END", 1)[0]
    return re.findall(r'"([^"]+)"', block)


def test_hip_lua_flags_equal_build_py():
    py = [f for f in B.COMMON if not f.startswith("-I")]
    assert _lua_flags() == py


def test_hip_lua_extra_flags_equal_build_py():
    text = (ROOT / "xmake" / "hip.lua").read_text()
    block = text.split("-- HIP_EXTRA_BEGIN", 1)[1].split("-- HIP_EXTRA_END", 1)[0]
    lua = {k: re.findall(r'"([^"]+)"', v) for k, v in re.findall(r'\["([^"]+)"\]\s*=\s*\{([^}]*)\}', block)}
    assert lua == B.EXTRA
    assert all((B.CSRC / k).is_file() for k in B.EXTRA)


def test_hip_lua_globs_cover_every_source():
    text = (ROOT / "xmake" / "hip.lua").read_text()
    assert 'add_files("../llaisys_amd/csrc/**.cpp", "../llaisys_amd/csrc/**.hip")' in text
    assert {p.suffix for p in B._sources()} <= {".cpp", ".hip"}
    # every kernel is this project's own: no GEMM library is linked
    assert "-lrocblas" not in Path(B.__file__).read_text() and "add_links" not in text


def test_root_xmake_has_amd_gpu_option_including_hip_lua():
    text = (ROOT / "xmake.lua").read_text()
    assert 'option("amd-gpu")' in text
    assert 'includes("xmake/hip.lua")' in text
