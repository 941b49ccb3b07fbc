"""The prefill's C ABI (include/pi05_prefill.h): every declared symbol is bound and exported, and
the host-only logic (geometry validation, device-memory plan, NULL handling) behaves.  No GPU
compute: only entry points that never touch HIP are called."""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from pi05_infer import _ext

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pi05_prefill.h")


@pytest.fixture(scope="module")
def lib():
    return _ext.load_prefix_library()


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return sorted(set(re.findall(r"\b(pi05_[a-z_0-9]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_functions() == sorted(_ext.PREFIX_EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", _ext.PREFIX_LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (pi05_\w+)", out))
    for name in header_functions():
        assert hasattr(lib, name) and name in exported, name


def test_default_dims_are_gemma_2b(lib):
    d = _ext.prefix_default_dims()
    assert (d.width, d.depth, d.num_heads, d.num_kv_heads, d.head_dim, d.mlp_dim) == (2048, 18, 8, 1, 256, 16384)
    assert (d.batch, d.prefix_len, d.skip_last_layer) == (1, 968, 1)
    assert d.rms_eps == np.float32(1e-6) and d.rope_theta == 10000.0
    _ext.prefix_check_dims(d)


@pytest.mark.parametrize(
    "field, value, msg",
    [("width", 1024, "width 2048"), ("mlp_dim", 4096, "mlp_dim 16384"), ("num_kv_heads", 2, "1 KV head"),
     ("depth", 0, "depth"), ("batch", 0, "batch"), ("prefix_len", 0, "prefix_len"), ("skip_last_layer", 2, "skip_last_layer")],
)
def test_invalid_dims_rejected_with_message(lib, field, value, msg):
    d = _ext.prefix_default_dims()
    setattr(d, field, value)
    with pytest.raises(_ext.Pi05Error) as e:
        _ext.prefix_check_dims(d)
    assert msg in str(e.value)
    assert _ext.prefix_device_bytes(d) == 0


def test_device_bytes_covers_weights_and_activations(lib):
    d = _ext.prefix_default_dims()
    need = 18 * (2560 * 2048 + 2048 * 2048 + 32768 * 2048 + 2048 * 16384) * 2  # packed bf16 weights (3.96 GB)
    need += 18 * 2 * 2048 * 4  # fp32 norm weights
    M = 968
    need += M * (3 * 2048 + 2560 + 2048 + 32768 + 16384) * 2  # h, n, y, q|k|v, attention out, gate|up, GeGLU out
    need += 992 * 8 * 256 * 2 + 2 * 992 * 256 * 2  # attention q fragments and K/V blocks (P padded to 992)
    need += 4 * 968 * 8 * (256 + 2) * 4  # 4 key splits (61 workgroups x 4 fill 244 CUs): fp32 partial O, max, sum
    need += 4 * 968 * 2048 * 4  # down_proj split-K fp32 partials (4 slices)
    got = _ext.prefix_device_bytes(d)
    assert need <= got <= need + 80 * 2**20  # + GEMM workspace and small tables
    d.batch = 2
    assert _ext.prefix_device_bytes(d) > got


def test_null_handles_and_pointers(lib):
    assert lib.pi05_prefix_destroy(None) == 0
    assert lib.pi05_prefix_bind_layer(None, 0, *([None] * 9)) == -1
    assert lib.pi05_prefix_refresh_weights(None, None) == -1
    assert lib.pi05_prefix_embed_tokens(None, None, 1, None, 1, None, None) == -1
    assert lib.pi05_prefix_forward(None, None, None, None, None, 0, 256, None) == -1
    assert lib.pi05_prefix_create(None, None) == -1
    bad = _ext.prefix_default_dims()
    bad.head_dim = 64
    h = ctypes.c_void_p()
    assert lib.pi05_prefix_create(ctypes.byref(bad), ctypes.byref(h)) == -1
    assert b"head_dim" in lib.pi05_prefix_last_error(None)
