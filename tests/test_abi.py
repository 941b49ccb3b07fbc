"""The C ABI library: it loads, exports every symbol include/pi05_denoise.h declares, and its
host-only logic (validation, schedule, sinusoid, RoPE frequencies) agrees with the oracle.
No GPU compute here: only entry points that never touch HIP are called."""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest
import torch

from oracle import denoise_oracle as O
from pi05_infer import _ext

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pi05_denoise.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_ext.LIB_PATH):
        import importlib.util

        spec = importlib.util.spec_from_file_location("build_lib", os.path.join(ROOT, "pi05-infer_amd", "build_lib.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return _ext.load_library()


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pi05_[a-z_0-9]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_functions() == sorted(_ext.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    for name in header_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _ext.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (pi05_\w+)", out))
    assert set(header_functions()) <= exported
    assert lib.pi05_abi_version() == _ext.ABI_VERSION


def test_default_dims_are_the_reference_geometry(lib):
    d = _ext.default_dims()
    assert (d.width, d.depth, d.num_heads, d.num_kv_heads, d.head_dim, d.mlp_dim) == (1024, 18, 8, 1, 256, 4096)
    assert (d.action_dim, d.action_horizon, d.batch, d.prefix_len, d.num_steps) == (32, 50, 1, 968, 10)
    assert d.rms_eps == np.float32(1e-6) and d.rope_theta == 10000.0
    _ext.check_dims(d)


@pytest.mark.parametrize(
    "field,value,msg",
    [
        ("width", 2048, "width"),
        ("num_heads", 16, "num_heads"),
        ("num_kv_heads", 2, "num_kv_heads"),
        ("head_dim", 128, "head_dim"),
        ("mlp_dim", 8192, "mlp_dim"),
        ("action_dim", 7, "action_dim"),
        ("action_horizon", 10, "action_horizon"),
        ("depth", 0, "depth"),
        ("batch", 0, "batch"),
        ("prefix_len", 0, "prefix_len"),
        ("num_steps", 0, "num_steps"),
        ("num_steps", 33, "num_steps"),
        ("rms_eps", -1.0, "rms_eps"),
    ],
)
def test_invalid_dims_rejected_with_message(lib, field, value, msg):
    d = _ext.default_dims()
    setattr(d, field, value)
    with pytest.raises(_ext.Pi05Error) as ei:
        _ext.check_dims(d)
    assert ei.value.code == -1 and msg in str(ei.value)
    assert _ext.device_bytes(d) == 0


def test_device_bytes_covers_weights_and_cache(lib):
    d = _ext.default_dims()
    need = 622_854_144  # 18 layers of bf16 expert weights
    need += 2 * 18 * 992 * 256 * 2  # prefix K and V cache (P padded to 992)
    need += 10 * 37 * 3072 * 4  # modulation table
    # per-(step, layer) activation slices of the persistent schedule (rows padded to 64 per
    # sample): GeGLU output, q and o, residual stream before and after attention, and the two
    # modulated copies g = bf16(h * (1 + scale)) that the folded adaRMSNorm GEMMs consume
    need += 10 * 18 * 64 * (4096 + 2 * 2048 + 3 * 1024) * 2 + 10 * 19 * 64 * 1024 * 2
    # shift . W^T per (step, layer): 2560 q|k|v + 2 x 4096 gate|up columns, fp32
    need += 10 * 18 * (2560 + 2 * 4096) * 4
    # per-(step, layer) split partials: attention (9 key splits x 25 row blocks x 16 rows x 256
    # fp32) and the down_proj K quarters (4 x 64 tiles x 64 rows x 16 fp32)
    need += 10 * 18 * (9 * 25 * 16 * 256 + 4 * 64 * 64 * 16) * 4
    # completion flags: (steps + 1) x (depth + 1) x 7 phases x 16 replicas x 512 words
    need += 11 * 19 * 7 * 16 * 512 * 4
    got = _ext.device_bytes(d)
    assert need <= got <= need + 64 * 2**20
    d8 = _ext.default_dims()
    d8.batch = 8
    assert _ext.device_bytes(d8) > got


def test_largest_dims_fit_the_kernel_32bit_offsets(lib):
    """pi05_check_dims rejects dims whose largest per-(step, layer) slice reaches 2^31 bytes (the
    persistent kernel's buffer offsets are 32-bit).  At the largest accepted dims (64 samples,
    16384 prefix tokens) the 1600 two-token row blocks fill the 256 workgroups with one key split
    each, so the largest windows are the GeGLU rows (64 * 64 rows x 4096 bf16 = 32 MiB) and the
    attention partials (1 split x 1600 row blocks x 16 rows x 256 fp32 = 25 MiB); the most key
    splits (16, at 16384 prefix tokens) occur at batches of at most 2, whose partials are
    16 x 50 x 16 x 256 fp32 = 12.5 MiB.  The plan's total size grows with the batch."""
    d = _ext.default_dims()
    d.batch, d.prefix_len, d.num_steps = 64, 16384, 32
    _ext.check_dims(d)
    assert 64 * 64 * 4096 * 2 == 32 * 2**20 < 2**31
    assert 1 * 64 * 25 * 16 * 256 * 4 < 2**31 and 16 * 2 * 25 * 16 * 256 * 4 < 2**31
    big = _ext.device_bytes(d)
    d.batch = 2
    _ext.check_dims(d)
    assert _ext.device_bytes(d) < big


def test_null_handles_and_pointers_are_invalid(lib):
    vp = ctypes.c_void_p
    assert lib.pi05_bind_layer(None, 0, *([None] * 11)) == -1
    assert lib.pi05_bind_heads(None, *([None] * 10)) == -1
    assert lib.pi05_refresh_weights(None, None) == -1
    assert lib.pi05_prime_prefix(None, None, None, 0, 256, None, None) == -1
    assert lib.pi05_denoise(None, None, None, None) == -1
    assert lib.pi05_bench_kernel(None, 0, 0, 1, None) == -1
    assert lib.pi05_release_graph(None) == -1
    assert lib.pi05_ctx_destroy(None) == 0
    assert lib.pi05_launches_per_step(None) == 0
    assert lib.pi05_last_error(None)
    assert lib.pi05_ctx_create(None, None) == -1
    bad = _ext.default_dims()
    bad.head_dim = 64
    h = vp()
    assert lib.pi05_ctx_create(ctypes.byref(bad), ctypes.byref(h)) == -1
    assert b"head_dim" in lib.pi05_last_error(None)


@pytest.mark.parametrize("n", list(range(1, 33)))
def test_host_schedule_matches_oracle(lib, n):
    assert torch.equal(_ext.euler_schedule(n), O.euler_timesteps(n))


def test_schedule_rejects_bad_counts(lib):
    with pytest.raises(_ext.Pi05Error):
        _ext.euler_schedule(0)


@pytest.mark.parametrize("t", [1.0, 0.9, 0.5, 0.1, 0.0, 0.3333333432674408])
def test_host_time_embedding_matches_oracle(lib, t):
    got = _ext.time_embedding(_ext.default_dims(), t)
    ref = O.sinusoidal_time_embedding(torch.tensor([t], dtype=torch.float32), 1024, 4e-3, 4.0)[0]
    assert torch.max((got - ref).abs()).item() <= 1.2e-7


def test_host_rope_inv_freq_matches_oracle(lib):
    got = _ext.rope_inv_freq(_ext.default_dims())
    ref = O.rope_inv_freq(256, 10000.0)
    assert torch.max((got - ref).abs() / ref).item() <= 1.2e-7
