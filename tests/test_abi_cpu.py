"""C-ABI checks that need no GPU: the library loads, exports every entry point
declared in include/vdx_sampler.h, lays out vdx_sampler_config exactly as the
Pascal TVdxSamplerConfig record (src/VindexLLM.Sampler.pas:26-34 under {$A8},
src/VindexLLM.Defines.inc:13), and fails loudly when no GPU is present."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vdx_sampler.h")


def _lib():
    from vindexllm_amd import build, sampler

    if not os.path.exists(build.LIB):
        build.build_library()
    return sampler.load_library()


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vdx_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    L = _lib()
    names = _declared_functions()
    assert len(names) >= 14
    for n in names:
        assert hasattr(L, n), n
    # the Python mirror binds exactly the declared set
    from vindexllm_amd import sampler
    assert sorted(sampler._SIGNATURES) == names


def test_config_layout_matches_pascal_record(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "vdx_sampler.h"\n'
        "int main(void){printf(\"%zu %zu %zu %zu %zu %zu %zu %zu\\n\", sizeof(vdx_sampler_config),"
        "offsetof(vdx_sampler_config,temperature),offsetof(vdx_sampler_config,top_k),"
        "offsetof(vdx_sampler_config,top_p),offsetof(vdx_sampler_config,min_p),"
        "offsetof(vdx_sampler_config,repeat_penalty),offsetof(vdx_sampler_config,repeat_window),"
        "offsetof(vdx_sampler_config,seed));return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    assert [int(x) for x in out] == [32, 0, 4, 8, 12, 16, 20, 24]
    from vindexllm_amd import TVdxSamplerConfig
    assert C.sizeof(TVdxSamplerConfig) == 32
    assert [getattr(TVdxSamplerConfig, f).offset for f, _ in TVdxSamplerConfig._fields_] == \
        [0, 4, 8, 12, 16, 20, 24]


def test_default_config_matches_reference():
    # TVdxSampler.DefaultConfig (Sampler.pas:100-109); UTest.Sampler.pas:79-86
    _lib()
    from vindexllm_amd import TVdxSampler
    c = TVdxSampler.DefaultConfig()
    assert (c.Temperature, c.TopK, c.TopP, c.MinP, c.RepeatPenalty, c.RepeatWindow, c.Seed) == \
        (0.0, 0, 1.0, 0.0, 1.0, 64, 0)


def test_version_string():
    _lib()
    from vindexllm_amd import version
    assert "gfx950" in version()


def test_create_fails_loudly_without_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    _lib()
    from vindexllm_amd import TVdxSampler, VdxSamplerError
    with pytest.raises(VdxSamplerError) as e:
        TVdxSampler(0, 4)
    assert e.value.code == -2 and "device" in str(e.value)


def test_missing_library_raises(monkeypatch, tmp_path):
    from vindexllm_amd import build, sampler
    monkeypatch.setattr(build, "LIB", str(tmp_path / "absent.so"))
    monkeypatch.setattr(sampler, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        sampler.load_library()


def test_lmhead_argument_errors_need_no_gpu():
    # argument validation runs before any HIP call and reports through
    # vdx_sampler_last_error(NULL)
    L = _lib()
    buf = (C.c_uint8 * 64)()
    base = C.addressof(buf)
    al = (base + 15) & ~15
    hid = C.c_void_p(al)
    cases = [
        (C.c_void_p(al), hid, 1, 100, 1024, "multiple of 32"),    # in_dim
        (C.c_void_p(al + 4), hid, 1, 256, 1024, "aligned"),       # weights alignment
        (None, hid, 1, 256, 1024, "required"),                    # weights
        (C.c_void_p(al), hid, 0, 256, 1024, "rows > 0"),          # rows
    ]
    rc = L.vdx_lmhead_q4_0(C.c_void_p(al), hid, 2, 256, 1024, C.c_void_p(al), 1024, None, None)
    assert rc == -1 and "scratch" in L.vdx_sampler_last_error(None).decode()
    for w, h, rows, d, v, msg in cases:
        rc = L.vdx_lmhead_q4_0(w, h, rows, d, v, C.c_void_p(al), v, C.c_void_p(al), None)
        assert rc == -1
        assert msg in L.vdx_sampler_last_error(None).decode()
    # the general entry point: an unknown weight type is unsupported; the norm
    # needs the scratch copy even for one row
    rc = L.vdx_lmhead(C.c_void_p(al), 0, hid, None, C.c_float(1e-6), 1, 256, 1024, C.c_void_p(al), 1024,
                      C.c_void_p(al), None)
    assert rc == -3 and "weight type" in L.vdx_sampler_last_error(None).decode()
    rc = L.vdx_lmhead(C.c_void_p(al), 8, hid, hid, C.c_float(1e-6), 1, 256, 1024, C.c_void_p(al), 1024,
                      None, None)
    assert rc == -1 and "scratch" in L.vdx_sampler_last_error(None).decode()


def test_lmhead_packed_bytes_needs_no_gpu():
    # the packed size: 64-row groups (the last padded) of whole rows
    from vindexllm_amd import VDX_LMHEAD_PACKED, lmhead_packed_bytes
    from vindexllm_amd.sampler import VdxSamplerError
    assert lmhead_packed_bytes(2, 2560, 262144) == 262144 * 80 * 18
    assert lmhead_packed_bytes(8, 2560, 262144 + 1) == (262144 + 64) * 80 * 34
    assert lmhead_packed_bytes(1, 256, 1) == 64 * 256 * 2
    for bad in ((3, 2560, 10), (2, 100, 10), (2, 2560, 0), (2 | VDX_LMHEAD_PACKED << 1, 256, 1)):
        with pytest.raises(VdxSamplerError):
            lmhead_packed_bytes(*bad)
