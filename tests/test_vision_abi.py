"""The vision tower's C ABI (include/pi05_siglip.h): every declared symbol is bound and exported,
and the host-only logic (geometry validation, device-memory plan, NULL handling) behaves.  No GPU
compute: only entry points that never touch HIP are called."""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from pi05_infer import _ext

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pi05_siglip.h")


@pytest.fixture(scope="module")
def lib():
    return _ext.load_prefix_library()


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return sorted(set(re.findall(r"\b(pi05_vision_[a-z_0-9]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_functions() == sorted(_ext.VISION_EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", _ext.PREFIX_LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (pi05_\w+)", out))
    for name in header_functions():
        assert hasattr(lib, name) and name in exported, name


def test_default_dims_are_siglip_so400m(lib):
    d = _ext.vision_default_dims()
    assert (d.width, d.depth, d.num_heads, d.mlp_dim, d.patch, d.image, d.channels, d.proj_dim) == \
        (1152, 27, 16, 4304, 14, 224, 3, 2048)
    assert d.n_images == 3 and d.ln_eps == np.float32(1e-6) and d.out_scale == 1.0
    _ext.vision_check_dims(d)


@pytest.mark.parametrize(
    "field, value, msg",
    [("width", 1024, "width 1152"), ("mlp_dim", 4096, "mlp_dim 4304"), ("patch", 16, "patch 14"), ("image", 448, "image 224"),
     ("depth", 0, "depth"), ("n_images", 0, "n_images"), ("ln_eps", 0.0, "ln_eps"), ("out_scale", -1.0, "out_scale")],
)
def test_invalid_dims_rejected_with_message(lib, field, value, msg):
    d = _ext.vision_default_dims()
    setattr(d, field, value)
    with pytest.raises(_ext.Pi05Error) as e:
        _ext.vision_check_dims(d)
    assert msg in str(e.value)
    assert _ext.vision_device_bytes(d) == 0


def test_device_bytes_covers_weights_and_activations(lib):
    d = _ext.vision_default_dims()
    W, I, P, S = 1152, 4304, 2048, 256
    Ip = 4352  # the MLP dim padded for 16-byte-aligned split-K slices of fc2
    need = 27 * (4 * W * W + I * W + W * Ip) * 2  # packed bf16 q|k|v, out, fc1, fc2 (0.8 GB)
    need += 27 * (3 * W + W + I + W + 4 * W) * 4  # fp32 biases and LayerNorm parameters
    need += (W * 588 + W + S * W + 2 * W + P) * 4 + P * W * 2  # patch/position embeddings, post-LN, projector
    M = 3 * S
    need += M * (4 * W + 3 * W + Ip) * 2  # h, n, y, attention out, q|k|v, fc1 out
    need += max(8 * M * W, 3 * M * Ip) * 4  # fp32 split-K partials: out_proj / fc2 (up to 8 slices), fc1 (up to 3)
    need += M * (588 + W) * 4  # fp32 patches and patch-embedding output
    got = _ext.vision_device_bytes(d)
    assert need <= got <= need + 40 * 2**20  # + GEMM workspace
    d.n_images = 6
    assert _ext.vision_device_bytes(d) > got


def test_null_handles_and_pointers(lib):
    assert lib.pi05_vision_destroy(None) == 0
    assert lib.pi05_vision_bind_layer(None, 0, *([None] * 16)) == -1
    assert lib.pi05_vision_bind_heads(None, *([None] * 7)) == -1
    assert lib.pi05_vision_refresh_weights(None, None) == -1
    assert lib.pi05_vision_forward(None, None, None, None) == -1
    assert lib.pi05_vision_create(None, None) == -1
    bad = _ext.vision_default_dims()
    bad.num_heads = 12
    h = ctypes.c_void_p()
    assert lib.pi05_vision_create(ctypes.byref(bad), ctypes.byref(h)) == -1
    assert b"16 heads" in lib.pi05_vision_last_error(None)
