"""C-ABI checks that need no GPU: the library loads, exports every function
include/g3attn.h declares, keeps gemma3_config's layout, and fails loudly
(NULL + message) when no device is present."""
import ctypes as C
import os
import shutil
import subprocess

import numpy as np
import pytest

from helpers import REPO, O, g3attn

G = g3attn()
REF_HDR = "/root/reference/gemma3.h"


def test_library_exports_every_declared_function():
    names = G.declared_functions()
    assert len(names) >= 18
    lib = C.CDLL(G.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_kernel_shim_is_hip_code_object():
    """The kernels are compiled into the library for gfx950 (no CPU path)."""
    data = open(G.LIB_PATH, "rb").read()
    assert b"gfx950" in data
    assert b"decode_kernel" in data and b"rope_write_kernel" in data


def test_default_config_matches_reference_constants():
    c = G.default_config()
    assert (c.num_layers, c.num_heads, c.num_kv_heads, c.head_dim) == (34, 8, 4, 256)
    assert (c.max_context, c.sliding_window) == (8192, 1024)
    assert c.rmsnorm_eps == np.float32(1e-6)
    assert (c.rope_theta_local, c.rope_theta_global) == (10000.0, 1000000.0)
    assert (c.vocab_size, c.hidden_size, c.intermediate_size) == (262208, 2560, 10240)
    if os.path.exists(REF_HDR):
        text = open(REF_HDR).read()
        for key, val in (("NUM_LAYERS", 34), ("NUM_HEADS", 8), ("NUM_KV_HEADS", 4),
                         ("HEAD_DIM", 256), ("SLIDING_WINDOW", 1024), ("DEFAULT_CONTEXT", 8192)):
            assert f"GEMMA3_{key}" in text
            line = [l for l in text.splitlines() if l.startswith(f"#define GEMMA3_{key} ")][0]
            assert int(line.split()[2]) == val


def test_global_layer_pattern():
    """gemma3.h:347-350: layers 5, 11, 17, 23, 29 of 34 are global."""
    glob = [l for l in range(34) if G.is_global_layer(l)]
    assert glob == [5, 11, 17, 23, 29]
    assert glob == [l for l in range(34) if O.is_global_layer(l)]


@pytest.mark.skipif(not os.path.exists(REF_HDR) or not shutil.which("gcc"),
                    reason="reference header not present on this machine")
def test_config_layout_equals_gemma3_config(tmp_path):
    """g3attn_config is gemma3_config field for field (a caller may cast)."""
    src = tmp_path / "layout.c"
    fields = ["vocab_size", "hidden_size", "intermediate_size", "num_layers", "num_heads",
              "num_kv_heads", "head_dim", "max_context", "sliding_window", "rmsnorm_eps",
              "rope_theta_local", "rope_theta_global"]
    checks = "\n".join(
        f"_Static_assert(offsetof(gemma3_config, {f}) == offsetof(g3attn_config, {f}), \"{f}\");"
        for f in fields)
    src.write_text(f'#include <stddef.h>\n#include "gemma3.h"\n#include "g3attn.h"\n'
                   f"_Static_assert(sizeof(gemma3_config) == sizeof(g3attn_config), \"size\");\n"
                   f"{checks}\nint main(void) {{ return 0; }}\n")
    subprocess.run(["gcc", "-std=c11", "-fsyntax-only", "-I/root/reference",
                    f"-I{os.path.join(REPO, 'include')}", str(src)], check=True)


def test_rope_precompute_matches_oracle_bitwise():
    for theta in (10000.0, 1e6):
        a = G.rope_precompute(4096, theta)
        b = O.rope_table(4096, theta)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _gpu_present():
    return os.path.exists("/dev/kfd")


@pytest.mark.skipif(_gpu_present(), reason="checks the no-device failure path")
def test_create_without_device_returns_null_with_message():
    t = O.rope_table(16, 1e4)
    with pytest.raises(G.G3AttnError) as e:
        G.Context(G.default_config(max_context=16), 16, t, t)
    assert "device" in str(e.value).lower()


@pytest.mark.skipif(_gpu_present(), reason="checks the no-device failure path")
def test_gqa_without_device_raises():
    q = np.zeros(2048, np.float32)
    kv = np.zeros(4 * 1024, np.float32)
    with pytest.raises(G.G3AttnError):
        G.gqa(q, kv, kv, 8, 4, 4)


def test_invalid_shapes_rejected_before_device_use():
    t = O.rope_table(16, 1e4)
    for bad in (dict(head_dim=128), dict(num_heads=6), dict(num_heads=8, num_kv_heads=1),
                dict(num_layers=0), dict(sliding_window=0)):
        cfg = G.default_config(max_context=16, **bad)
        h = G.lib().g3attn_create(C.byref(cfg), 16, t.ctypes.data, t.ctypes.data)
        assert not h
        assert G.last_error()


def test_create_needs_both_tables_or_neither():
    t = O.rope_table(16, 1e4)
    cfg = G.default_config(max_context=16)
    assert not G.lib().g3attn_create(C.byref(cfg), 16, t.ctypes.data, None)
    assert "RoPE table" in G.last_error()
    assert not G.lib().g3attn_create(C.byref(cfg), 16, None, t.ctypes.data)


def test_injected_create_failure(monkeypatch):
    """G3ATTN_FAULT=create fails g3attn_create before any device use, with
    its cause in the message; the list is comma-separated, sites match whole."""
    t = O.rope_table(16, 1e4)
    cfg = G.default_config(max_context=16)
    for val in ("create", "upload,create", "create,forward"):
        monkeypatch.setenv("G3ATTN_FAULT", val)
        assert not G.lib().g3attn_create(C.byref(cfg), 16, t.ctypes.data, t.ctypes.data)
        assert "injected" in G.last_error(), val
    if not _gpu_present():
        monkeypatch.setenv("G3ATTN_FAULT", "creat,createx,upload")
        assert not G.lib().g3attn_create(C.byref(cfg), 16, t.ctypes.data, t.ctypes.data)
        assert "injected" not in G.last_error() and "device" in G.last_error()


def test_upload_rope_rejects_a_null_context():
    t = O.rope_table(16, 1e4)
    assert G.lib().g3attn_upload_rope(None, t, t, 16, 256) == G.ERR_INVALID_ARG
    assert "null" in G.last_error()


@pytest.mark.skipif(not os.path.exists("/root/reference/gemma3_transformer.c"),
                    reason="reference sources not present on this machine")
def test_backend_hook_declares_the_engines_functions():
    """include/g3backend.h declares exactly the backend functions that
    gemma3_transformer.c declares under USE_MPS (:17-31), and
    libg3backend.so exports them."""
    import re
    src = open("/root/reference/gemma3_transformer.c").read()
    block = src[src.index("#ifdef USE_MPS"):]
    block = block[:block.index("#endif")]
    want = set(re.findall(r"\b(gemma3_metal_\w+)\s*\(", block))
    hdr = re.sub(r"/\*.*?\*/", "", open(os.path.join(REPO, "include", "g3backend.h")).read(), flags=re.S)
    have = set(re.findall(r"\b(gemma3_metal_\w+)\s*\(", hdr))
    assert len(want) == 7 and want <= have and have - want == {"gemma3_metal_available"}
    lib = C.CDLL(os.path.join(REPO, "gemma3.c_amd", "lib", "libg3backend.so"))
    for name in have:
        assert hasattr(lib, name), name
