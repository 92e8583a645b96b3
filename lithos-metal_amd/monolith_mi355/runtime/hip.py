"""ctypes binding of ``libmi355.so`` — the C ABI declared in ``include/lithos_mi355.h``.

This module replaces the reference's nanobind ``_native`` module (``runtime/src/native.mm:13-95``): it loads the
shared library built from ``lithos-metal_amd/csrc`` and turns every non-zero return code into a ``RuntimeError``
carrying ``mi_last_error()`` (the reference raises C++ ``std::runtime_error`` as Python exceptions,
``runtime/src/metal_core.mm:49,67,106,117``). There is no fallback: a missing library raises at load time.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path
from typing import Optional

LIB_NAME = "libmi355.so"
_PKG_ROOT = Path(__file__).resolve().parents[2]          # lithos-metal_amd/
LIB_PATH = Path(os.environ.get("LITHOS_MI355_LIB", _PKG_ROOT / "lib" / LIB_NAME))

MI_FMT = {"nvfp4": 1, "int4_affine": 2, "bf16": 3, "fp8_e4m3": 4}
MI_EPI = {None: 0, "none": 0, "residual": 1, "silu_mul": 2, "silu_mul_rounded": 3}


class MiDeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("arch", C.c_char * 64), ("compute_units", C.c_int32),
                ("clock_khz", C.c_int32), ("hbm_bytes", C.c_int64), ("lds_bytes_per_block", C.c_int32),
                ("warp_size", C.c_int32)]


class MiGemvDesc(C.Structure):
    _fields_ = [("format", C.c_int32), ("n", C.c_int32), ("k", C.c_int32), ("m", C.c_int32),
                ("w", C.c_void_p), ("row_scale", C.c_void_p), ("x", C.c_void_p), ("ldx", C.c_int32),
                ("y", C.c_void_p), ("ldy", C.c_int32), ("epilogue", C.c_int32), ("residual", C.c_void_p),
                ("ldr", C.c_int32), ("norm_w", C.c_void_p), ("eps", C.c_float), ("groups", C.c_void_p),
                ("max_groups", C.c_int32), ("top_k", C.c_int32), ("x_per_slot", C.c_int32),
                ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t), ("out_f32", C.c_int32),
                ("gnorm_w", C.c_void_p), ("gnorm_z", C.c_void_p), ("ld_gnorm_z", C.c_int32), ("gnorm_eps", C.c_float),
                ("shared_expert", C.c_int32), ("shared_epilogue", C.c_int32), ("route_logits", C.c_void_p),
                ("route_experts", C.c_int32), ("route_top_k", C.c_int32), ("route_renorm", C.c_int32),
                ("route_gate_col", C.c_int32), ("route_ids", C.c_void_p), ("route_weights", C.c_void_p),
                ("group_max_pairs", C.c_int32), ("route_ld", C.c_int32), ("conv_w", C.c_void_p),
                ("conv_in", C.c_void_p), ("conv_out_state", C.c_void_p), ("conv_out", C.c_void_p),
                ("conv_row0", C.c_int32), ("conv_channels", C.c_int32), ("ld_conv", C.c_int32),
                ("conv_step", C.c_void_p), ("conv_done", C.c_void_p), ("next_norm_w", C.c_void_p),
                ("next_x", C.c_void_p), ("ld_next_x", C.c_int32), ("next_eps", C.c_float)]


class MiGdnDesc(C.Structure):
    _fields_ = [("t", C.c_int32), ("k_heads", C.c_int32), ("v_heads", C.c_int32), ("dk", C.c_int32), ("dv", C.c_int32),
                ("conv_width", C.c_int32), ("proj", C.c_void_p), ("ld_proj", C.c_int32), ("z_off", C.c_int32),
                ("q_off", C.c_int32), ("k_off", C.c_int32), ("v_off", C.c_int32), ("ab", C.c_void_p),
                ("ld_ab", C.c_int32), ("a_off", C.c_int32), ("b_off", C.c_int32), ("conv_w", C.c_void_p),
                ("neg_exp_a", C.c_void_p), ("dt_bias", C.c_void_p), ("norm_w", C.c_void_p), ("conv_in", C.c_void_p),
                ("conv_out", C.c_void_p), ("rec_in", C.c_void_p), ("rec_out", C.c_void_p), ("y", C.c_void_p),
                ("ld_y", C.c_int32), ("eps", C.c_float), ("defer_norm", C.c_int32), ("commit", C.c_int32),
                ("t_dev", C.c_void_p), ("done", C.c_void_p), ("step", C.c_void_p), ("pre", C.c_void_p),
                ("ld_pre", C.c_int32)]


MI_KV_INT8, MI_KV_BF16 = 0, 1


class MiGqaDesc(C.Structure):
    _fields_ = [("t", C.c_int32), ("heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("rotary_dim", C.c_int32), ("pos", C.c_int32), ("ctx_max", C.c_int32), ("gate", C.c_int32),
                ("qk_norm", C.c_int32), ("proj", C.c_void_p), ("ld_proj", C.c_int32), ("rope_cos", C.c_void_p),
                ("rope_sin", C.c_void_p), ("q_norm", C.c_void_p), ("k_norm", C.c_void_p), ("eps", C.c_float),
                ("scaling", C.c_float), ("k_codes", C.c_void_p), ("k_scales", C.c_void_p), ("v_codes", C.c_void_p),
                ("v_scales", C.c_void_p), ("y", C.c_void_p), ("ld_y", C.c_int32), ("workspace", C.c_void_p),
                ("workspace_bytes", C.c_size_t), ("pos_dev", C.c_void_p),
                ("done", C.c_void_p), ("kv_dtype", C.c_int32), ("gate_src", C.c_void_p), ("ld_gate", C.c_int32)]


class MiNormDesc(C.Structure):
    _fields_ = [("t", C.c_int32), ("k", C.c_int32), ("h", C.c_void_p), ("ldh", C.c_int32), ("stat", C.c_void_p),
                ("stat_parts", C.c_int32), ("w", C.c_void_p), ("x", C.c_void_p), ("ldx", C.c_int32),
                ("eps", C.c_float)]


class MiMoeRouteDesc(C.Structure):
    _fields_ = [("t", C.c_int32), ("n_experts", C.c_int32), ("top_k", C.c_int32), ("renorm", C.c_int32),
                ("logits", C.c_void_p), ("ld_logits", C.c_int32), ("ids", C.c_void_p), ("weights", C.c_void_p),
                ("groups", C.c_void_p), ("max_groups", C.c_int32), ("shared_expert", C.c_int32),
                ("shared_gate_col", C.c_int32), ("pairs_per_record", C.c_int32)]


class MiMoeCombineDesc(C.Structure):
    _fields_ = [("t", C.c_int32), ("hidden", C.c_int32), ("top_k", C.c_int32), ("h", C.c_void_p), ("ldh", C.c_int32),
                ("weights", C.c_void_p), ("shared", C.c_void_p), ("ld_shared", C.c_int32), ("shared_gate", C.c_void_p),
                ("ld_gate", C.c_int32), ("residual", C.c_void_p), ("ldr", C.c_int32), ("out", C.c_void_p),
                ("ldo", C.c_int32), ("next_norm_w", C.c_void_p), ("next_x", C.c_void_p), ("ld_next_x", C.c_int32),
                ("next_eps", C.c_float)]


class MiStepState(C.Structure):
    """``mi_step_state``: the reference's StepStateLayout order (``core/step_state.py:38-63``) at t_max 16,
    gamma_max 15."""
    _u = C.c_uint32
    _fields_ = [("step", _u), ("position", _u), ("kv_len", _u), ("t_this_step", _u),
                ("pending_tokens", C.c_int32 * 16), ("rng_lo", _u), ("rng_hi", _u), ("anchor", C.c_int32),
                ("gamma", _u), ("draft_tokens", C.c_int32 * 15), ("confidence", C.c_float * 15),
                ("verify_len", _u), ("accepted", _u), ("checkpoint_index", _u), ("drafter_ctx_len", _u),
                ("done", _u), ("error", _u), ("ring_head", _u), ("ring_tail", _u), ("prefill_left", _u),
                ("n_inject", _u), ("stop_at", _u), ("n_chain", _u), ("pad_", _u * 2)]


class MiEmbedDesc(C.Structure):
    _fields_ = [("t", C.c_int32), ("vocab", C.c_int32), ("hidden", C.c_int32), ("tokens", C.c_void_p),
                ("table", C.c_void_p), ("out", C.c_void_p), ("ldo", C.c_int32), ("t16", C.c_int32)]


class MiArgmaxDesc(C.Structure):
    _fields_ = [("t", C.c_int32), ("vocab", C.c_int32), ("logits", C.c_void_p), ("ld", C.c_int32),
                ("f32", C.c_int32), ("ids", C.c_void_p), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t)]


class MiSampleDesc(C.Structure):
    _fields_ = [("t", C.c_int32), ("vocab", C.c_int32), ("logits", C.c_void_p), ("ld", C.c_int32), ("ids", C.c_void_p),
                ("temperature", C.c_float), ("top_p", C.c_float), ("min_p", C.c_float), ("top_k", C.c_int32),
                ("topp_in_topk", C.c_int32), ("seed", C.c_uint64), ("step", C.c_uint32), ("state", C.c_void_p),
                ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t)]


class MiAdvanceDesc(C.Structure):
    _fields_ = [("state", C.c_void_p), ("tokens", C.c_void_p), ("ring", C.c_void_p), ("ring_cap", C.c_uint32),
                ("ctx_cap", C.c_uint32), ("n_eos", C.c_int32), ("eos", C.c_int32 * 8), ("host_ctl", C.c_void_p)]


class MiVerifySelectDesc(C.Structure):
    _fields_ = [("state", C.c_void_p), ("drafts", C.c_void_p), ("conf", C.c_void_p), ("gamma", C.c_uint32),
                ("t_max", C.c_uint32), ("mode", C.c_uint32), ("threshold", C.c_float), ("cost", C.c_float * 16),
                ("conf_log", C.c_void_p), ("log_cap", C.c_uint32), ("ctx_cap", C.c_uint32), ("lm", C.c_uint32)]


class MiAcceptScanDesc(C.Structure):
    _fields_ = [("state", C.c_void_p), ("tokens", C.c_void_p), ("ring", C.c_void_p), ("ring_cap", C.c_uint32),
                ("ctx_cap", C.c_uint32), ("lm", C.c_uint32), ("n_eos", C.c_int32), ("eos", C.c_int32 * 8),
                ("log", C.c_void_p), ("log_cap", C.c_uint32), ("host_ctl", C.c_void_p)]


class MiRunnerDesc(C.Structure):
    _fields_ = [("graph_exec", C.c_void_p), ("stream", C.c_void_p), ("state", C.c_void_p), ("ring", C.c_void_p),
                ("ring_capacity", C.c_uint32), ("host_ctl", C.c_void_p), ("max_launches", C.c_uint32),
                ("launches_per_batch", C.c_uint32), ("in_flight", C.c_uint32), ("max_tokens", C.c_uint64),
                ("tokens", C.c_void_p), ("tokens_capacity", C.c_uint64), ("n_tokens", C.c_uint64),
                ("state_ring_tail", C.c_void_p), ("state_done", C.c_void_p), ("state_error", C.c_void_p)]


class MiRunnerStats(C.Structure):
    _fields_ = [("launches", C.c_uint64), ("batches", C.c_uint64), ("tokens", C.c_uint64), ("wall_ms", C.c_double),
                ("gpu_ms", C.c_double), ("launch_ms", C.c_double), ("wait_ms", C.c_double),
                ("host_busy_ms", C.c_double), ("done", C.c_uint32), ("error", C.c_uint32)]


# name -> (restype, argtypes); every int-returning entry point is error-checked
_VP, _I32, _SZ, _F = C.c_void_p, C.c_int32, C.c_size_t, C.c_float
class MiKernelAttrs(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("max_threads_per_block", "static_lds_bytes", "registers", "scratch_bytes",
                                         "wave_size")]


SIGNATURES = {
    "mi_version": (C.c_char_p, []),
    "mi_last_error": (C.c_int, [C.c_char_p, _SZ]),
    "mi_device_count": (C.c_int, [C.POINTER(_I32)]),
    "mi_device_info_get": (C.c_int, [_I32, C.POINTER(MiDeviceInfo)]),
    "mi_set_device": (C.c_int, [_I32]),
    "mi_malloc": (C.c_int, [C.POINTER(_VP), _SZ]),
    "mi_free": (C.c_int, [_VP]),
    "mi_memcpy_h2d": (C.c_int, [_VP, _VP, _SZ, _VP]),
    "mi_memcpy_d2h": (C.c_int, [_VP, _VP, _SZ, _VP]),
    "mi_memcpy_d2d": (C.c_int, [_VP, _VP, _SZ, _VP]),
    "mi_memset": (C.c_int, [_VP, _I32, _SZ, _VP]),
    "mi_stream_create": (C.c_int, [C.POINTER(_VP)]),
    "mi_stream_destroy": (C.c_int, [_VP]),
    "mi_stream_synchronize": (C.c_int, [_VP]),
    "mi_event_create": (C.c_int, [C.POINTER(_VP)]),
    "mi_event_destroy": (C.c_int, [_VP]),
    "mi_event_record": (C.c_int, [_VP, _VP]),
    "mi_event_synchronize": (C.c_int, [_VP]),
    "mi_event_elapsed_ms": (C.c_int, [_VP, _VP, C.POINTER(_F)]),
    "mi_graph_begin": (C.c_int, [_VP]),
    "mi_graph_end": (C.c_int, [_VP, C.POINTER(_VP)]),
    "mi_graph_launch": (C.c_int, [_VP, _VP]),
    "mi_graph_destroy": (C.c_int, [_VP]),
    "mi_pack_bytes": (_SZ, [_I32, _I32, _I32]),
    "mi_gemv_workspace_bytes": (_SZ, [C.POINTER(MiGemvDesc)]),
    "mi_gemv": (C.c_int, [C.POINTER(MiGemvDesc), _VP]),
    "mi_gemv_noalloc": (C.c_int, [C.POINTER(MiGemvDesc), _VP]),
    "mi_gemv_chain_workspace_bytes": (_SZ, [C.POINTER(MiGemvDesc), _I32]),
    "mi_gemv_chain": (C.c_int, [C.POINTER(MiGemvDesc), _I32, _VP, _SZ, _VP]),
    "mi_gemv_chain_error": (C.c_int, [_VP, _VP, C.POINTER(C.c_uint32)]),
    "mi_gemv_noalloc_scratch_bytes": (_SZ, []),
    "mi_gemv_plan": (C.c_int, [C.POINTER(MiGemvDesc), C.POINTER(_I32)]),
    "mi_dequant": (C.c_int, [_I32, _VP, _VP, _I32, _I32, _VP, _VP]),
    "mi_gdn_step": (C.c_int, [C.POINTER(MiGdnDesc), _VP]),
    "mi_rmsnorm_stat": (C.c_int, [C.POINTER(MiNormDesc), _VP]),
    "mi_norm_apply": (C.c_int, [C.POINTER(MiNormDesc), _VP]),
    "mi_gqa_workspace_bytes": (_SZ, [C.POINTER(MiGqaDesc)]),
    "mi_gqa_decode": (C.c_int, [C.POINTER(MiGqaDesc), _VP]),
    "mi_moe_route": (C.c_int, [C.POINTER(MiMoeRouteDesc), _VP]),
    "mi_moe_combine": (C.c_int, [C.POINTER(MiMoeCombineDesc), _VP]),
    "mi_embed": (C.c_int, [C.POINTER(MiEmbedDesc), _VP]),
    "mi_argmax_workspace_bytes": (_SZ, [C.POINTER(MiArgmaxDesc)]),
    "mi_argmax": (C.c_int, [C.POINTER(MiArgmaxDesc), _VP]),
    "mi_sample_workspace_bytes": (_SZ, [C.POINTER(MiSampleDesc)]),
    "mi_sample": (C.c_int, [C.POINTER(MiSampleDesc), _VP]),
    "mi_advance": (C.c_int, [C.POINTER(MiAdvanceDesc), _VP]),
    "mi_verify_select": (C.c_int, [C.POINTER(MiVerifySelectDesc), _VP]),
    "mi_accept_scan": (C.c_int, [C.POINTER(MiAcceptScanDesc), _VP]),
    "mi_runner_run": (C.c_int, [C.POINTER(MiRunnerDesc), C.POINTER(MiRunnerStats)]),
    "mi_host_alloc": (_VP, [_SZ]),
    "mi_host_free": (C.c_int, [_VP]),
    "mi_library_compile": (C.c_int, [C.c_char_p, C.POINTER(C.c_char_p), _I32, _I32, C.POINTER(_VP), C.POINTER(_SZ)]),
    "mi_code_free": (C.c_int, [_VP]),
    "mi_library_load": (C.c_int, [_VP, _SZ, C.POINTER(_VP)]),
    "mi_library_release": (C.c_int, [_VP]),
    "mi_kernel_get": (C.c_int, [_VP, C.c_char_p, C.POINTER(_VP)]),
    "mi_kernel_info": (C.c_int, [_VP, C.POINTER(MiKernelAttrs)]),
    "mi_launch": (C.c_int, [_VP, _VP, _SZ, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.c_uint32, _VP]),
    "mi_buf_from_file": (C.c_int, [C.c_char_p, C.c_uint64, _SZ, C.POINTER(_VP)]),
}


class MiError(RuntimeError):
    pass


_lib: Optional[C.CDLL] = None


def load(path: Optional[os.PathLike] = None) -> C.CDLL:
    """Load (once) and type the library. Raises if it is missing — the product path has no CPU fallback."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise MiError(f"{p} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                      f"or `python lithos-metal_amd/build.py`")
    # torch first, so that this library binds to the HIP runtime torch loads and the two share devices and
    # streams: with hiprtc used before torch initialised the GPU, this library's calls saw no device
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    buf = C.create_string_buffer(512)
    load().mi_last_error(buf, 512)
    return buf.value.decode(errors="replace")


def call(name: str, *args) -> int:
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise MiError(f"{name} failed ({rc}): {last_error()}")
    return rc


def device_info(device: int = 0) -> MiDeviceInfo:
    info = MiDeviceInfo()
    call("mi_device_info_get", device, C.byref(info))
    return info


def ptr(t) -> int:
    """Device address of a tensor-like (``.data_ptr()``), an int, or None → 0."""
    if t is None:
        return 0
    if isinstance(t, int):
        return t
    return int(t.data_ptr())


def stream_handle(stream=None) -> Optional[int]:
    """A HIP stream handle: an int, a ``torch.cuda.Stream``, or None → torch's current stream when torch has one."""
    if stream is None:
        try:
            import torch
            if torch.cuda.is_available():
                return int(torch.cuda.current_stream().cuda_stream)
        except ImportError:
            pass
        return None
    if isinstance(stream, int):
        return stream
    return int(stream.cuda_stream)


class Event:
    """A HIP event pair helper for timing work on one stream (``Queue.profile``'s per-dispatch timestamps,
    ``runtime/src/metal_core.mm:157-210``)."""

    def __init__(self):
        h = C.c_void_p()
        call("mi_event_create", C.byref(h))
        self.h = h

    def record(self, stream=None):
        call("mi_event_record", self.h, stream_handle(stream))

    def synchronize(self):
        call("mi_event_synchronize", self.h)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        call("mi_event_elapsed_ms", self.h, end.h, C.byref(ms))
        return float(ms.value)

    def __del__(self):
        try:
            if _lib is not None and self.h:
                _lib.mi_event_destroy(self.h)
        except Exception:
            pass


class Graph:
    """Stream capture → replayable graph: the reference's pre-encoded ICB (``runtime/src/metal_core.h:106-116``)."""

    def __init__(self, stream):
        self.stream = stream_handle(stream)
        self.exec = None

    def __enter__(self):
        call("mi_graph_begin", self.stream)
        return self

    def __exit__(self, *exc):
        h = C.c_void_p()
        call("mi_graph_end", self.stream, C.byref(h))
        self.exec = h
        return False

    def launch(self, stream=None):
        call("mi_graph_launch", self.exec, stream_handle(stream) if stream is not None else self.stream)

    def __del__(self):
        try:
            if _lib is not None and self.exec:
                _lib.mi_graph_destroy(self.exec)
        except Exception:
            pass
