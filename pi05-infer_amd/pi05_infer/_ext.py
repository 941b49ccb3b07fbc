"""ctypes bindings of ``libpi05_denoise.so`` (the C ABI in ``include/pi05_denoise.h``) and
``libpi05_prefix.so`` (``include/pi05_prefill.h`` and ``include/pi05_siglip.h``, loaded on first
use, so a denoise-only process never loads hipBLASLt).

The shared libraries are built in-tree next to this file (``build_lib.py``).  There is no
fallback: if a library is missing or fails to load, every entry point of it raises.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import torch

LIB_NAME = "libpi05_denoise.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
PREFIX_LIB_NAME = "libpi05_prefix.so"
PREFIX_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), PREFIX_LIB_NAME)
ABI_VERSION = 1

PI05_OK = 0
SCHEDULES = {"persistent": 0, "graph": 1}
ERROR_NAMES = {-1: "PI05_E_INVALID", -2: "PI05_E_STATE", -3: "PI05_E_HIP", -4: "PI05_E_NOMEM", -5: "PI05_E_NODEVICE"}

# every exported symbol of include/pi05_denoise.h
EXPORTED_SYMBOLS = (
    "pi05_abi_version",
    "pi05_default_dims",
    "pi05_check_dims",
    "pi05_ctx_device_bytes",
    "pi05_ctx_create",
    "pi05_ctx_destroy",
    "pi05_last_error",
    "pi05_bind_layer",
    "pi05_bind_heads",
    "pi05_refresh_weights",
    "pi05_get_adarms_table",
    "pi05_prime_prefix",
    "pi05_get_step_invariants",
    "pi05_denoise",
    "pi05_denoise_status",
    "pi05_debug_set_spin_limit",
    "pi05_debug_set_epoch",
    "pi05_debug_skew_placement_check",
    "pi05_release_graph",
    "pi05_set_schedule",
    "pi05_get_schedule",
    "pi05_launches_per_step",
    "pi05_bench_kernel",
    "pi05_adarms_table_noalloc",
    "pi05_euler_schedule",
    "pi05_time_embedding",
    "pi05_rope_inv_freq",
)

# every exported symbol of include/pi05_prefill.h
PREFIX_EXPORTED_SYMBOLS = (
    "pi05_prefix_default_dims",
    "pi05_prefix_check_dims",
    "pi05_prefix_device_bytes",
    "pi05_prefix_create",
    "pi05_prefix_destroy",
    "pi05_prefix_last_error",
    "pi05_prefix_bind_layer",
    "pi05_prefix_refresh_weights",
    "pi05_prefix_embed_tokens",
    "pi05_prefix_status",
    "pi05_prefix_forward",
)

# every exported symbol of include/pi05_siglip.h
VISION_EXPORTED_SYMBOLS = (
    "pi05_vision_default_dims",
    "pi05_vision_check_dims",
    "pi05_vision_device_bytes",
    "pi05_vision_create",
    "pi05_vision_destroy",
    "pi05_vision_last_error",
    "pi05_vision_bind_layer",
    "pi05_vision_bind_heads",
    "pi05_vision_refresh_weights",
    "pi05_vision_forward",
)


class Pi05Error(RuntimeError):
    """A non-zero status from the engine's C ABI."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {message}")
        self.code = code


class Pi05Dims(ctypes.Structure):
    _fields_ = [
        ("width", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("mlp_dim", ctypes.c_int32),
        ("action_dim", ctypes.c_int32),
        ("action_horizon", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("prefix_len", ctypes.c_int32),
        ("num_steps", ctypes.c_int32),
        ("rms_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
        ("time_min_period", ctypes.c_double),
        ("time_max_period", ctypes.c_double),
    ]


class Pi05PrefixDims(ctypes.Structure):
    _fields_ = [
        ("width", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("mlp_dim", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("prefix_len", ctypes.c_int32),
        ("rms_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
        ("skip_last_layer", ctypes.c_int32),
    ]


class Pi05VisionDims(ctypes.Structure):
    _fields_ = [
        ("width", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("mlp_dim", ctypes.c_int32),
        ("patch", ctypes.c_int32),
        ("image", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("proj_dim", ctypes.c_int32),
        ("n_images", ctypes.c_int32),
        ("ln_eps", ctypes.c_float),
        ("out_scale", ctypes.c_float),
    ]


_lib: Optional[ctypes.CDLL] = None
_prefix_lib: Optional[ctypes.CDLL] = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and type the engine library; raises if it is absent or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{LIB_NAME} not found at {path}; build it first (python pi05-infer_amd/build_lib.py). "
            "There is no fallback implementation."
        )
    lib = ctypes.CDLL(path)
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    dims_p = ctypes.POINTER(Pi05Dims)
    sig = {
        "pi05_abi_version": (i32, []),
        "pi05_default_dims": (None, [dims_p]),
        "pi05_check_dims": (i32, [dims_p]),
        "pi05_ctx_device_bytes": (ctypes.c_size_t, [dims_p]),
        "pi05_ctx_create": (i32, [dims_p, ctypes.POINTER(vp)]),
        "pi05_ctx_destroy": (i32, [vp]),
        "pi05_last_error": (ctypes.c_char_p, [vp]),
        "pi05_bind_layer": (i32, [vp, i32] + [vp] * 11),
        "pi05_bind_heads": (i32, [vp] + [vp] * 10),
        "pi05_refresh_weights": (i32, [vp, vp]),
        "pi05_get_adarms_table": (i32, [vp, vp, vp]),
        "pi05_prime_prefix": (i32, [vp, ctypes.POINTER(vp), ctypes.POINTER(vp), i64, i64, vp, vp]),
        "pi05_get_step_invariants": (i32, [vp, vp, vp, vp, vp]),
        "pi05_denoise": (i32, [vp, vp, vp, vp]),
        "pi05_denoise_status": (i32, [vp, vp]),
        "pi05_debug_set_spin_limit": (i32, [vp, i32]),
        "pi05_debug_set_epoch": (i32, [vp, ctypes.c_uint32]),
        "pi05_debug_skew_placement_check": (i32, [vp, i32]),
        "pi05_release_graph": (i32, [vp]),
        "pi05_set_schedule": (i32, [vp, i32]),
        "pi05_get_schedule": (i32, [vp]),
        "pi05_launches_per_step": (i32, [vp]),
        "pi05_bench_kernel": (i32, [vp, i32, i32, i32, vp]),
        "pi05_adarms_table_noalloc": (i32, [dims_p, vp, vp, vp, vp, ctypes.POINTER(vp), ctypes.POINTER(vp), vp, vp]),
        "pi05_euler_schedule": (i32, [i32, vp]),
        "pi05_time_embedding": (i32, [dims_p, ctypes.c_float, vp]),
        "pi05_rope_inv_freq": (i32, [dims_p, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.pi05_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_NAME} ABI {lib.pi05_abi_version()} != expected {ABI_VERSION}")
    _lib = lib
    return lib


def load_prefix_library(path: str = PREFIX_LIB_PATH) -> ctypes.CDLL:
    """Load (once) and type the prefill / vision library; raises if it is absent."""
    global _prefix_lib
    if _prefix_lib is not None:
        return _prefix_lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{PREFIX_LIB_NAME} not found at {path}; build it first (python pi05-infer_amd/build_lib.py). "
            "There is no fallback implementation."
        )
    lib = ctypes.CDLL(path)
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    pdims_p = ctypes.POINTER(Pi05PrefixDims)
    vdims_p = ctypes.POINTER(Pi05VisionDims)
    sig = {
        "pi05_prefix_default_dims": (None, [pdims_p]),
        "pi05_prefix_check_dims": (i32, [pdims_p]),
        "pi05_prefix_device_bytes": (ctypes.c_size_t, [pdims_p]),
        "pi05_prefix_create": (i32, [pdims_p, ctypes.POINTER(vp)]),
        "pi05_prefix_destroy": (i32, [vp]),
        "pi05_prefix_last_error": (ctypes.c_char_p, [vp]),
        "pi05_prefix_bind_layer": (i32, [vp, i32] + [vp] * 9),
        "pi05_prefix_refresh_weights": (i32, [vp, vp]),
        "pi05_prefix_embed_tokens": (i32, [vp, vp, i64, vp, i64, vp, vp]),
        "pi05_prefix_status": (i32, [vp, vp]),
        "pi05_prefix_forward": (i32, [vp, vp, vp, ctypes.POINTER(vp), ctypes.POINTER(vp), i64, i64, vp]),
        "pi05_vision_default_dims": (None, [vdims_p]),
        "pi05_vision_check_dims": (i32, [vdims_p]),
        "pi05_vision_device_bytes": (ctypes.c_size_t, [vdims_p]),
        "pi05_vision_create": (i32, [vdims_p, ctypes.POINTER(vp)]),
        "pi05_vision_destroy": (i32, [vp]),
        "pi05_vision_last_error": (ctypes.c_char_p, [vp]),
        "pi05_vision_bind_layer": (i32, [vp, i32] + [vp] * 16),
        "pi05_vision_bind_heads": (i32, [vp] + [vp] * 7),
        "pi05_vision_refresh_weights": (i32, [vp, vp]),
        "pi05_vision_forward": (i32, [vp, vp, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _prefix_lib = lib
    return lib


def _check(lib: ctypes.CDLL, rc: int, ctx: Optional[int]) -> None:
    if rc != PI05_OK:
        msg = lib.pi05_last_error(ctx)
        raise Pi05Error(rc, msg.decode() if msg else "")


def default_dims() -> Pi05Dims:
    lib = load_library()
    d = Pi05Dims()
    lib.pi05_default_dims(ctypes.byref(d))
    return d


def make_dims(geometry, batch: int, prefix_len: int, num_steps: int) -> Pi05Dims:
    g = geometry
    return Pi05Dims(
        g.width, g.depth, g.num_heads, g.num_kv_heads, g.head_dim, g.mlp_dim, g.action_dim, g.action_horizon,
        batch, prefix_len, num_steps, g.rms_eps, g.rope_theta, g.time_min_period, g.time_max_period,
    )


def check_dims(dims: Pi05Dims) -> None:
    """Validate dims without touching a GPU; raises Pi05Error(PI05_E_INVALID)."""
    lib = load_library()
    _check(lib, lib.pi05_check_dims(ctypes.byref(dims)), None)


def device_bytes(dims: Pi05Dims) -> int:
    return int(load_library().pi05_ctx_device_bytes(ctypes.byref(dims)))


def adarms_table_noalloc(dims: Pi05Dims, tin_w, tin_b, tout_w, tout_b, dense_w: Sequence[torch.Tensor],
                         dense_b: Sequence[torch.Tensor], out: torch.Tensor, stream=None) -> torch.Tensor:
    """pi05_adarms_table_noalloc: the modulation table from caller-owned fp32 device tensors into
    ``out`` ``[num_steps, 2*depth+1, 3W]`` fp32, with no device allocation by the library."""
    lib = load_library()
    n = 2 * dims.depth + 1
    if len(dense_w) != n or len(dense_b) != n:
        raise ValueError(f"need {n} dense weights and biases")
    dev = out.device
    f32 = torch.float32
    if tuple(out.shape) != (dims.num_steps, n, 3 * dims.width):
        raise ValueError("out shape mismatch")
    wp = (ctypes.c_void_p * n)(*[_ptr(t, f32, "dense_w", dev) for t in dense_w])
    bp = (ctypes.c_void_p * n)(*[_ptr(t, f32, "dense_b", dev) for t in dense_b])
    rc = lib.pi05_adarms_table_noalloc(ctypes.byref(dims), _ptr(tin_w, f32, "tin_w", dev), _ptr(tin_b, f32, "tin_b", dev),
                                       _ptr(tout_w, f32, "tout_w", dev), _ptr(tout_b, f32, "tout_b", dev), wp, bp,
                                       _ptr(out, f32, "out", dev), _stream_ptr(stream))
    _check(lib, rc, None)
    return out


def euler_schedule(num_steps: int) -> torch.Tensor:
    """Host-side Euler schedule of the engine ``[num_steps + 1]`` fp32."""
    lib = load_library()
    out = torch.empty(num_steps + 1, dtype=torch.float32)
    _check(lib, lib.pi05_euler_schedule(num_steps, out.data_ptr()), None)
    return out


def time_embedding(dims: Pi05Dims, t: float) -> torch.Tensor:
    """Host-side sinusoidal timestep embedding ``[width]`` fp32."""
    lib = load_library()
    out = torch.empty(dims.width, dtype=torch.float32)
    _check(lib, lib.pi05_time_embedding(ctypes.byref(dims), t, out.data_ptr()), None)
    return out


def rope_inv_freq(dims: Pi05Dims) -> torch.Tensor:
    """Host-side RoPE inverse frequencies ``[head_dim / 2]`` fp32."""
    lib = load_library()
    out = torch.empty(dims.head_dim // 2, dtype=torch.float32)
    _check(lib, lib.pi05_rope_inv_freq(ctypes.byref(dims), out.data_ptr()), None)
    return out


def _ptr(t: torch.Tensor, dtype: torch.dtype, name: str, device: torch.device) -> int:
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if t.device != device:
        raise ValueError(f"{name}: expected device {device}, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    return t.data_ptr()


def _stream_ptr(stream: Optional[torch.cuda.Stream]) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


class DenoiseContext:
    """One engine context: a (batch, prefix_len, num_steps) signature on the current device."""

    def __init__(self, geometry, batch: int, prefix_len: int, num_steps: int, device: torch.device):
        self.lib = load_library()
        self.geometry = geometry
        self.dims = make_dims(geometry, batch, prefix_len, num_steps)
        self.device = torch.device(device)
        _check(self.lib, self.lib.pi05_check_dims(ctypes.byref(self.dims)), None)
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _check(self.lib, self.lib.pi05_ctx_create(ctypes.byref(self.dims), ctypes.byref(handle)), None)
        self.handle = handle.value
        self._keepalive: list = []

    @property
    def signature(self) -> tuple[int, int, int]:
        return (self.dims.batch, self.dims.prefix_len, self.dims.num_steps)

    def _call(self, rc: int) -> None:
        _check(self.lib, rc, self.handle)

    def bind_layer(self, i: int, wq, wk, wv, wo, wgate, wup, wdown, ln1_w, ln1_b, ln2_w, ln2_b) -> None:
        bf, f32, dev = torch.bfloat16, torch.float32, self.device
        ptrs = [
            _ptr(wq, bf, "wq", dev), _ptr(wk, bf, "wk", dev), _ptr(wv, bf, "wv", dev), _ptr(wo, bf, "wo", dev),
            _ptr(wgate, bf, "wgate", dev), _ptr(wup, bf, "wup", dev), _ptr(wdown, bf, "wdown", dev),
            _ptr(ln1_w, f32, "ln1_w", dev), _ptr(ln1_b, f32, "ln1_b", dev),
            _ptr(ln2_w, f32, "ln2_w", dev), _ptr(ln2_b, f32, "ln2_b", dev),
        ]
        self._call(self.lib.pi05_bind_layer(self.handle, i, *ptrs))

    def bind_heads(self, norm_w, norm_b, in_w, in_b, out_w, out_b, tin_w, tin_b, tout_w, tout_b) -> None:
        f32, dev = torch.float32, self.device
        names = ("norm_w", "norm_b", "in_w", "in_b", "out_w", "out_b", "tin_w", "tin_b", "tout_w", "tout_b")
        ts = (norm_w, norm_b, in_w, in_b, out_w, out_b, tin_w, tin_b, tout_w, tout_b)
        self._call(self.lib.pi05_bind_heads(self.handle, *[_ptr(t, f32, n, dev) for t, n in zip(ts, names)]))

    def refresh_weights(self, stream=None) -> None:
        self._call(self.lib.pi05_refresh_weights(self.handle, _stream_ptr(stream)))

    def adarms_table(self, stream=None) -> torch.Tensor:
        d = self.dims
        out = torch.empty((d.num_steps, 2 * d.depth + 1, 3 * d.width), dtype=torch.float32, device=self.device)
        self._call(self.lib.pi05_get_adarms_table(self.handle, out.data_ptr(), _stream_ptr(stream)))
        return out

    def step_invariants(self, stream=None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """The primed step invariants in the reference's layout: RoPE positions int64 ``[B, A]``,
        key-valid uint8 ``[B, P + A]`` (prefix keys, then the action keys) and the number of padding
        slots of the context's key table marked valid (int32 ``[1]``, 0 for a correct table)."""
        d = self.dims
        pos = torch.empty((d.batch, d.action_horizon), dtype=torch.int64, device=self.device)
        valid = torch.empty((d.batch, d.prefix_len + d.action_horizon), dtype=torch.uint8, device=self.device)
        stray = torch.empty(1, dtype=torch.int32, device=self.device)
        self._call(self.lib.pi05_get_step_invariants(self.handle, pos.data_ptr(), valid.data_ptr(), stray.data_ptr(),
                                                     _stream_ptr(stream)))
        return pos, valid, stray

    def prime_prefix(self, k_layers: Sequence[torch.Tensor], v_layers: Sequence[torch.Tensor],
                     prefix_pad: torch.Tensor, stream=None) -> None:
        """k_layers/v_layers: per layer bf16 [B, 1, P, D] (or any view whose last dim is contiguous
        and whose batch/position strides are uniform across layers)."""
        d = self.dims
        if len(k_layers) != d.depth or len(v_layers) != d.depth:
            raise ValueError(f"expected {d.depth} K and V layers, got {len(k_layers)} / {len(v_layers)}")
        ref = k_layers[0]
        if ref.dim() != 4 or tuple(ref.shape) != (d.batch, 1, d.prefix_len, d.head_dim):
            raise ValueError(f"K layer shape {tuple(ref.shape)} != {(d.batch, 1, d.prefix_len, d.head_dim)}")
        bstride, rstride = ref.stride(0), ref.stride(2)
        for name, layers in (("K", k_layers), ("V", v_layers)):
            for i, t in enumerate(layers):
                if t.dtype != torch.bfloat16 or t.device != self.device:
                    raise TypeError(f"{name}[{i}] must be bf16 on {self.device}")
                if tuple(t.shape) != tuple(ref.shape) or t.stride(0) != bstride or t.stride(2) != rstride or t.stride(3) != 1:
                    raise ValueError(f"{name}[{i}] shape/strides differ from layer 0")
        pad = prefix_pad
        if pad.dtype == torch.bool:
            pad = pad.to(torch.uint8)
        if pad.dtype != torch.uint8 or tuple(pad.shape) != (d.batch, d.prefix_len):
            raise ValueError(f"prefix_pad must be bool/uint8 [{d.batch}, {d.prefix_len}]")
        pad = pad.to(self.device).contiguous()
        karr = (ctypes.c_void_p * d.depth)(*[t.data_ptr() for t in k_layers])
        varr = (ctypes.c_void_p * d.depth)(*[t.data_ptr() for t in v_layers])
        self._keepalive = [pad]
        self._call(self.lib.pi05_prime_prefix(self.handle, karr, varr, bstride, rstride, pad.data_ptr(), _stream_ptr(stream)))

    def denoise(self, x: torch.Tensor, trace: Optional[torch.Tensor] = None, stream=None) -> None:
        """In place: x [B, A, a] fp32 noise -> actions.  trace [steps, B, A, a] fp32 or None."""
        d = self.dims
        if tuple(x.shape) != (d.batch, d.action_horizon, d.action_dim):
            raise ValueError(f"x shape {tuple(x.shape)} != {(d.batch, d.action_horizon, d.action_dim)}")
        xp = _ptr(x, torch.float32, "x", self.device)
        tp = None
        if trace is not None:
            if tuple(trace.shape) != (d.num_steps, d.batch, d.action_horizon, d.action_dim):
                raise ValueError("trace shape mismatch")
            tp = _ptr(trace, torch.float32, "trace", self.device)
        self._call(self.lib.pi05_denoise(self.handle, xp, tp, _stream_ptr(stream)))

    def status(self, stream=None) -> None:
        """Wait for the stream; raise Pi05Error(PI05_E_HIP) if a denoise launch of this context
        timed out and was not reported yet (denoise itself only enqueues)."""
        self._call(self.lib.pi05_denoise_status(self.handle, _stream_ptr(stream)))

    def set_spin_limit(self, polls: int) -> None:
        """Test hook: polls after which a kernel wait gives up (0 = the default)."""
        self._call(self.lib.pi05_debug_set_spin_limit(self.handle, polls))

    def skew_placement_check(self, skew: int) -> None:
        """Test hook: perturb the kernel's XCD placement check (0 restores it)."""
        self._call(self.lib.pi05_debug_skew_placement_check(self.handle, int(skew)))

    def set_epoch(self, epoch: int) -> None:
        """Test hook: the epoch of the last finished persistent launch (the next runs as epoch + 1);
        lets a test cross the 2^31 wrap-around."""
        self._call(self.lib.pi05_debug_set_epoch(self.handle, epoch))

    def release_graph(self) -> None:
        self._call(self.lib.pi05_release_graph(self.handle))

    @property
    def schedule(self) -> str:
        """``"persistent"`` (one cooperative kernel per denoise) or ``"graph"`` (hipGraph of kernels)."""
        code = int(self.lib.pi05_get_schedule(self.handle))
        return {v: k for k, v in SCHEDULES.items()}[code]

    def set_schedule(self, name: str) -> None:
        """Switch schedule; the prefix must be primed again afterwards."""
        if name not in SCHEDULES:
            raise ValueError(f"schedule must be one of {sorted(SCHEDULES)}, got {name!r}")
        self._call(self.lib.pi05_set_schedule(self.handle, SCHEDULES[name]))

    KERNELS = ("step_io", "qkv_rope", "attention", "o_proj", "gate_up", "down")

    def bench_kernel(self, name: str, layer: int = 0, iters: int = 1, stream=None) -> None:
        """Enqueue ``iters`` launches of one step kernel (profiling; clobbers activations)."""
        self._call(self.lib.pi05_bench_kernel(self.handle, self.KERNELS.index(name), layer, iters, _stream_ptr(stream)))

    def launches_per_step(self) -> int:
        return int(self.lib.pi05_launches_per_step(self.handle))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.pi05_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------------------------------------ prefill


def _check_prefix(lib: ctypes.CDLL, rc: int, ctx: Optional[int]) -> None:
    if rc != PI05_OK:
        msg = lib.pi05_prefix_last_error(ctx)
        raise Pi05Error(rc, msg.decode() if msg else "")


def prefix_default_dims() -> Pi05PrefixDims:
    lib = load_prefix_library()
    d = Pi05PrefixDims()
    lib.pi05_prefix_default_dims(ctypes.byref(d))
    return d


def prefix_check_dims(dims: Pi05PrefixDims) -> None:
    lib = load_prefix_library()
    _check_prefix(lib, lib.pi05_prefix_check_dims(ctypes.byref(dims)), None)


def prefix_device_bytes(dims: Pi05PrefixDims) -> int:
    return int(load_prefix_library().pi05_prefix_device_bytes(ctypes.byref(dims)))


class PrefixContext:
    """One prefix-LM prefill context: a (batch, prefix_len) signature on the current device."""

    def __init__(self, dims: Pi05PrefixDims, device: torch.device):
        self.lib = load_prefix_library()
        self.dims = dims
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        _check_prefix(self.lib, self.lib.pi05_prefix_check_dims(ctypes.byref(self.dims)), None)
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _check_prefix(self.lib, self.lib.pi05_prefix_create(ctypes.byref(self.dims), ctypes.byref(handle)), None)
        self.handle = handle.value

    def _call(self, rc: int) -> None:
        _check_prefix(self.lib, rc, self.handle)

    def bind_layer(self, i: int, wq, wk, wv, wo, wgate, wup, wdown, ln1_w, ln2_w) -> None:
        bf, f32, dev = torch.bfloat16, torch.float32, self.device
        ptrs = [
            _ptr(wq, bf, "wq", dev), _ptr(wk, bf, "wk", dev), _ptr(wv, bf, "wv", dev), _ptr(wo, bf, "wo", dev),
            _ptr(wgate, bf, "wgate", dev), _ptr(wup, bf, "wup", dev), _ptr(wdown, bf, "wdown", dev),
            _ptr(ln1_w, f32, "ln1_w", dev), _ptr(ln2_w, f32, "ln2_w", dev),
        ]
        self._call(self.lib.pi05_prefix_bind_layer(self.handle, i, *ptrs))

    def refresh_weights(self, stream=None) -> None:
        self._call(self.lib.pi05_prefix_refresh_weights(self.handle, _stream_ptr(stream)))

    def embed_tokens(self, ids: torch.Tensor, table: torch.Tensor, stream=None) -> torch.Tensor:
        """``bf16(table[ids] * sqrt(W))`` for int32/int64 ids of any shape -> ``[*ids.shape, W]``.
        Enqueues only: device ids outside ``[0, vocab)`` give zero rows and are reported by the
        next call or by ``status()``; host ids are checked here, before the copy."""
        if ids.device.type == "cpu" and ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= table.shape[0]):
            raise Pi05Error(-1, "a token id is outside [0, vocab)")
        ids32 = ids.to(device=self.device, dtype=torch.int32).contiguous()
        tp = _ptr(table, torch.bfloat16, "table", self.device)
        out = torch.empty((*ids.shape, self.dims.width), dtype=torch.bfloat16, device=self.device)
        self._call(self.lib.pi05_prefix_embed_tokens(self.handle, ids32.data_ptr(), ids32.numel(), tp, table.shape[0],
                                                     out.data_ptr(), _stream_ptr(stream)))
        return out

    def status(self, stream=None) -> None:
        """Wait for the stream; raise if an earlier ``embed_tokens`` met a token id outside
        ``[0, vocab)`` that has not been reported yet."""
        self._call(self.lib.pi05_prefix_status(self.handle, _stream_ptr(stream)))

    def forward(self, embeds: torch.Tensor, prefix_pad: torch.Tensor, k_layers: Sequence[torch.Tensor],
                v_layers: Sequence[torch.Tensor], stream=None) -> None:
        """embeds [B, P, W] bf16, prefix_pad [B, P] bool/uint8 -> K/V written into k_layers / v_layers
        (per layer bf16 [B, 1, P, D] views with the same strides)."""
        d = self.dims
        if tuple(embeds.shape) != (d.batch, d.prefix_len, d.width):
            raise ValueError(f"embeds shape {tuple(embeds.shape)} != {(d.batch, d.prefix_len, d.width)}")
        ep = _ptr(embeds, torch.bfloat16, "embeds", self.device)
        pad = prefix_pad.to(torch.uint8) if prefix_pad.dtype == torch.bool else prefix_pad
        if pad.dtype != torch.uint8 or tuple(pad.shape) != (d.batch, d.prefix_len):
            raise ValueError(f"prefix_pad must be bool/uint8 [{d.batch}, {d.prefix_len}]")
        pad = pad.to(self.device).contiguous()
        if len(k_layers) != d.depth or len(v_layers) != d.depth:
            raise ValueError(f"expected {d.depth} K and V layers")
        ref = k_layers[0]
        if tuple(ref.shape) != (d.batch, 1, d.prefix_len, d.head_dim):
            raise ValueError(f"K layer shape {tuple(ref.shape)} != {(d.batch, 1, d.prefix_len, d.head_dim)}")
        bstride, rstride = ref.stride(0), ref.stride(2)
        for name, layers in (("K", k_layers), ("V", v_layers)):
            for i, t in enumerate(layers):
                if t.dtype != torch.bfloat16 or t.device != self.device:
                    raise TypeError(f"{name}[{i}] must be bf16 on {self.device}")
                if tuple(t.shape) != tuple(ref.shape) or t.stride(0) != bstride or t.stride(2) != rstride or t.stride(3) != 1:
                    raise ValueError(f"{name}[{i}] shape/strides differ from layer 0")
        karr = (ctypes.c_void_p * d.depth)(*[t.data_ptr() for t in k_layers])
        varr = (ctypes.c_void_p * d.depth)(*[t.data_ptr() for t in v_layers])
        self._pad = pad
        self._call(self.lib.pi05_prefix_forward(self.handle, ep, pad.data_ptr(), karr, varr, bstride, rstride,
                                                _stream_ptr(stream)))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.pi05_prefix_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------------------------------------ vision tower


def _check_vision(lib: ctypes.CDLL, rc: int, ctx: Optional[int]) -> None:
    if rc != PI05_OK:
        msg = lib.pi05_vision_last_error(ctx)
        raise Pi05Error(rc, msg.decode() if msg else "")


def vision_default_dims() -> Pi05VisionDims:
    lib = load_prefix_library()
    d = Pi05VisionDims()
    lib.pi05_vision_default_dims(ctypes.byref(d))
    return d


def vision_check_dims(dims: Pi05VisionDims) -> None:
    lib = load_prefix_library()
    _check_vision(lib, lib.pi05_vision_check_dims(ctypes.byref(dims)), None)


def vision_device_bytes(dims: Pi05VisionDims) -> int:
    return int(load_prefix_library().pi05_vision_device_bytes(ctypes.byref(dims)))


class VisionContext:
    """One SigLIP + projector context: an image count on the current device."""

    def __init__(self, dims: Pi05VisionDims, device: torch.device):
        self.lib = load_prefix_library()
        self.dims = dims
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        _check_vision(self.lib, self.lib.pi05_vision_check_dims(ctypes.byref(self.dims)), None)
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _check_vision(self.lib, self.lib.pi05_vision_create(ctypes.byref(self.dims), ctypes.byref(handle)), None)
        self.handle = handle.value

    def _call(self, rc: int) -> None:
        _check_vision(self.lib, rc, self.handle)

    def bind_layer(self, i: int, wq, bq, wk, bk, wv, bv, wo, bo, w1, b1, w2, b2, ln1_w, ln1_b, ln2_w, ln2_b) -> None:
        """Encoder layer i, every tensor bf16 (the reference's dtype for the encoder)."""
        names = ("wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "w1", "b1", "w2", "b2", "ln1_w", "ln1_b", "ln2_w", "ln2_b")
        ts = (wq, bq, wk, bk, wv, bv, wo, bo, w1, b1, w2, b2, ln1_w, ln1_b, ln2_w, ln2_b)
        ptrs = [_ptr(t, torch.bfloat16, n, self.device) for t, n in zip(ts, names)]
        self._call(self.lib.pi05_vision_bind_layer(self.handle, i, *ptrs))

    def bind_heads(self, patch_w, patch_b, pos, post_w, post_b, proj_w, proj_b) -> None:
        """Patch/position embeddings fp32, post_layernorm and projector bf16."""
        f32, bf, dev = torch.float32, torch.bfloat16, self.device
        ptrs = [_ptr(patch_w, f32, "patch_w", dev), _ptr(patch_b, f32, "patch_b", dev), _ptr(pos, f32, "pos", dev),
                _ptr(post_w, bf, "post_w", dev), _ptr(post_b, bf, "post_b", dev), _ptr(proj_w, bf, "proj_w", dev),
                _ptr(proj_b, bf, "proj_b", dev)]
        self._call(self.lib.pi05_vision_bind_heads(self.handle, *ptrs))

    def refresh_weights(self, stream=None) -> None:
        self._call(self.lib.pi05_vision_refresh_weights(self.handle, _stream_ptr(stream)))

    def forward(self, pixels: torch.Tensor, out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """pixels [N, 3, 224, 224] fp32 -> image embeddings [N, 256, proj_dim] bf16."""
        d = self.dims
        shape = (d.n_images, d.channels, d.image, d.image)
        if tuple(pixels.shape) != shape:
            raise ValueError(f"pixels shape {tuple(pixels.shape)} != {shape}")
        pp = _ptr(pixels, torch.float32, "pixels", self.device)
        n_patches = (d.image // d.patch) ** 2
        if out is None:
            out = torch.empty((d.n_images, n_patches, d.proj_dim), dtype=torch.bfloat16, device=self.device)
        elif tuple(out.shape) != (d.n_images, n_patches, d.proj_dim):
            raise ValueError(f"out shape {tuple(out.shape)} != {(d.n_images, n_patches, d.proj_dim)}")
        op = _ptr(out, torch.bfloat16, "out", self.device)
        self._call(self.lib.pi05_vision_forward(self.handle, pp, op, _stream_ptr(stream)))
        return out

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.pi05_vision_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
