"""Loader for ``libmlcg_hip.so``, the gfx950 kernel library.

The library exposes a plain C ABI (``include/mlcg_hip.h``); this module binds
it with :mod:`ctypes`.  PyTorch is imported first so that the HIP runtime
already mapped by torch (soname ``libamdhip64.so.7``) is the one the library
resolves against: the kernels then run on torch's streams and device memory.

There is no fallback: if the shared object is missing or a call returns a
non-zero status, a :class:`RuntimeError` is raised (the same error class the
reference's native operator raises, ``radius.cu:7-9``; the reference defers a
failed build to first use with ``DelayedError``, ``radius.py:35-49`` -- this
module does the same: importing never fails, calling does).
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch  # noqa: F401  (maps the HIP runtime before the library loads)

LIB_NAME = "libmlcg_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

_c = ctypes
_P = _c.c_void_p
_I64 = _c.c_int64
_I32 = _c.c_int
_F32 = _c.c_float
_F64 = _c.c_double
_U64 = _c.c_uint64

# name -> argtypes (all functions return int status unless listed in _RESTYPES)
_SIGNATURES = {
    "mlcg_version": [],
    "mlcg_frame_ptr_from_batch": [_P, _I64, _I64, _P, _P],
    "mlcg_radius_count": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _P, _P, _P],
    "mlcg_radius_count_f64": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _P, _P, _P],
    "mlcg_radius_fill_f64": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _I64, _I64, _P,
                             _P, _P],
    "mlcg_radius_fill_f16": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _I64, _I64, _P,
                             _P, _P],
    "mlcg_radius_fill_bf16": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _I64, _I64, _P,
                              _P, _P],
    "mlcg_radius_rowptr_f16": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _P, _P, _P],
    "mlcg_radius_rowptr_bf16": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _P, _P, _P],
    "mlcg_exclusion_pair_to_ptr": [_P, _I64, _I64, _P, _P],
    "mlcg_radius_workspace_bytes": [_I64],
    "mlcg_radius_rowptr": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _P, _P, _P, _P],
    "mlcg_radius_rowptr_f64": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _P, _P, _P,
                               _P],
    "mlcg_radius_graph": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _P, _I64, _I64, _P,
                          _P, _I64, _I64, _P, _P, _P, _P, _P],
    "mlcg_radius_graph_f64": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _I64, _I64, _P,
                              _P, _P, _P],
    "mlcg_scan_workspace_ints": [_I64],
    "mlcg_exclusive_scan2_i32": [_P, _P, _I64, _P, _P, _P, _P],
    "mlcg_exclusive_scan2_i32_noalloc": [_P, _P, _I64, _P, _P, _P],
    "mlcg_radius_fill": [_P, _P, _P, _I64, _F64, _I32, _I64, _P, _P, _P, _P, _I64, _I64, _P,
                         _P, _I64, _I64, _P, _P, _P, _P],
    "mlcg_pair_reverse_map": [_P, _I64, _P, _I64, _P, _P, _P, _P],
    "mlcg_filter_fwd": [_P, _P, _I64, _P, _I64, _I32, _P, _P, _F32, _I32, _I32, _F32, _F32,
                        _I32, _F32, _F32, _I32, _P, _P, _P, _I32, _I32, _P, _P, _P, _P],
    "mlcg_filter_bwd_workspace_floats": [_I64, _I32],
    "mlcg_filter_bwd": [_P, _P, _I64, _P, _I64, _I32, _P, _P, _F32, _I32, _I32, _F32, _F32,
                        _I32, _F32, _F32, _I32, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _P,
                        _P, _I64, _I32, _P],
    "mlcg_filter_bwd_cfconv": [_P, _P, _I64, _P, _I64, _I32, _P, _P, _F32, _I32, _I32, _F32,
                               _F32, _I32, _F32, _F32, _I32, _P, _P, _P, _I32, _P, _P, _P, _P,
                               _P, _P, _P, _P, _P, _P, _P, _I64, _I32, _P],
    "mlcg_rbf_param_grad_workspace_floats": [_I64, _I32],
    "mlcg_rbf_param_grad": [_P, _P, _I64, _I32, _P, _P, _F32, _I32, _I32, _F32, _F32, _P, _I32,
                            _P, _P, _I32, _P, _P, _P, _I64, _P],
    "mlcg_cfconv_gather": [_P, _P, _I32, _P, _P, _P, _I64, _I32, _P, _P],
    "mlcg_cfconv_gather_bwd": [_P, _P, _P, _P, _I32, _P, _P, _P, _I64, _I32, _P, _P, _I32,
                               _P],
    "mlcg_cfconv_gather_tangent": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I32, _P, _P],
    "mlcg_cfconv_gather_rev2": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I32, _P, _P,
                                _P, _P],
    "mlcg_pair_ddot": [_P, _P, _P, _I64, _P, _I64, _P, _F32, _P, _P],
    "mlcg_pair_forces": [_P, _P, _P, _P, _P, _P, _I64, _I32, _P, _P],
    "mlcg_segment_sum_f64": [_P, _P, _I64, _P, _P],
    "mlcg_cfconv_gather_f64": [_P, _P, _P, _P, _P, _I64, _I32, _P, _P],
    "mlcg_segment_sum": [_P, _I64, _P, _I64, _P, _P],
    "mlcg_node_gemm": [_P, _I64, _I32, _P, _I32, _P, _P, _I32, _I32, _P, _P, _P, _P, _P, _P,
                       _P, _P],
    "mlcg_node_gemm2": [_P, _I64, _I32, _P, _I32, _P, _P, _I32, _I32, _P, _P, _P, _P, _P, _P,
                        _P, _P, _P, _P, _P, _P, _P],
    "mlcg_node_weight_image_bytes": [],
    "mlcg_node_weight_images": [_P, _P, _I32, _P, _P],
    "mlcg_out_forward": [_P, _I64, _I32, _I32, _P, _P, _P, _P, _I32, _I32, _P, _P, _P, _P, _P,
                         _P],
    "mlcg_out_rev2_workspace_floats": [_I64, _I32],
    "mlcg_out_rev2": [_P, _P, _I64, _I32, _I32, _P, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _P,
                      _P, _P, _P, _I64, _P],
    "mlcg_node_tmm_workspace_floats": [_I64],
    "mlcg_node_tmm_batch_workspace_floats": [_I64, _I32],
    "mlcg_node_tmm_batch": [_P, _I32, _I64, _I32, _I32, _P, _I64, _P],
    "mlcg_node_tmm": [_P, _P, _P, _P, _I64, _I32, _I32, _P, _P, _P, _I64, _P],
    "mlcg_type_sum_workspace_floats": [_I64, _I32],
    "mlcg_type_sum": [_P, _P, _I64, _I32, _I32, _P, _P, _P, _I64, _P],
    "mlcg_prior_order": [_I32],
    "mlcg_prior_num_params": [_I32, _I32],
    "mlcg_prior_terms": [_I32, _I32, _P, _P, _I64, _I64, _P, _I32, _P, _P, _P],
    "mlcg_prior_terms_f64": [_I32, _I32, _P, _P, _I64, _I64, _P, _I32, _P, _P, _P],
    "mlcg_prior_gather_forces": [_P, _P, _P, _I64, _I32, _P, _P],
    "mlcg_prior_gather_forces_f64": [_P, _P, _P, _I64, _I32, _P, _P],
    "mlcg_prior_pair_records_ints": [_I64, _I64],
    "mlcg_prior_pair_records": [_P, _I64, _I64, _P, _I32, _P, _P, _I64, _P, _P],
    "mlcg_prior_repulsion": [_P, _I64, _P, _I64, _I64, _P, _P, _P, _P, _I32, _P, _P],
    "mlcg_langevin_baoa": [_P, _P, _P, _P, _P, _I64, _F32, _F32, _F32, _U64, _P, _P, _P],
    "mlcg_langevin_baoa_f64": [_P, _P, _P, _P, _P, _I64, _F64, _F64, _F64, _U64, _P, _P, _P],
    "mlcg_langevin_b": [_P, _P, _P, _I64, _F32, _P, _P],
    "mlcg_langevin_b_f64": [_P, _P, _P, _I64, _F64, _P, _P],
    "mlcg_philox_normals": [_U64, _I64, _I64, _P, _P],
    "mlcg_math_eval": [_I32, _P, _I64, _P, _P],
    "mlcg_numerics_flags": [_P, _I32, _P],
    "mlcg_embedding_gather": [_P, _I32, _I32, _P, _I64, _P, _P],
    "mlcg_stream_read": [_P, _I64, _I32, _I32, _P, _P],
    "mlcg_stream_copy": [_P, _P, _I64, _I32, _I32, _P],
    "mlcg_mfma_loop": [_I32, _I64, _I32, _P, _P],
    "mlcg_mfma_loop_flops_per_wave_iter": [_I32],
    "mlcg_copy_batch": [_P, _P, _P, _I32, _P],
    "mlcg_sum_arrays": [_P, _I32, _I64, _P, _P],
    "mlcg_mse_workspace_floats": [_I64],
    "mlcg_mse_mean": [_P, _P, _I64, _P, _P, _I64, _P],
    "mlcg_mse_mean_backward": [_P, _P, _P, _I64, _P, _P],
}
_RESTYPES = {"mlcg_version": _c.c_char_p, "mlcg_scan_workspace_ints": _I64,
             "mlcg_radius_workspace_bytes": _I64,
             "mlcg_filter_bwd_workspace_floats": _I64, "mlcg_node_tmm_workspace_floats": _I64,
             "mlcg_node_tmm_batch_workspace_floats": _I64,
             "mlcg_out_rev2_workspace_floats": _I64,
             "mlcg_rbf_param_grad_workspace_floats": _I64,
             "mlcg_type_sum_workspace_floats": _I64, "mlcg_node_weight_image_bytes": _I64,
             "mlcg_mse_workspace_floats": _I64, "mlcg_prior_pair_records_ints": _I64,
             "mlcg_mfma_loop_flops_per_wave_iter": _I64}

STATUS = {
    0: "MLCG_OK",
    1: "MLCG_ERR_ARGUMENT",
    2: "MLCG_ERR_LAUNCH",
    3: "MLCG_ERR_CAPACITY",
    4: "MLCG_ERR_UNSUPPORTED",
}

_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None


def exported_symbols():
    """Names of every entry point this binding expects the library to export."""
    return list(_SIGNATURES)


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise RuntimeError if it is absent."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        _load_error = (
            f"{LIB_PATH} not found: build it with `make -C mlcg_amd/csrc` or "
            "`python -c 'import __graft_entry__ as g; g.build()'`"
        )
        raise RuntimeError(_load_error)
    lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, _I32)
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


class LaunchTimer:
    """Brackets launches of selected entry points with HIP events recorded on
    torch's current stream (the stream every wrapper launches on), so the
    device time of each launch can be read after a synchronisation.

    ``watch`` is a set of entry-point names, or None for every entry point.
    A wrapper may pass the algorithmic work of a launch (bytes or FLOPs, as
    the wrapper knows the shapes and the epilogue); ``work()`` sums it.
    """

    def __init__(self, watch=None):
        self.watch = None if watch is None else set(watch)
        self.events = {}
        self.amounts = {}

    def wants(self, name: str) -> bool:
        return self.watch is None or name in self.watch

    def record(self, name: str, work=None):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        self.events.setdefault(name, []).append((start, end))
        if work is not None:
            self.amounts[name] = self.amounts.get(name, 0) + work
        return start, end

    def summary(self):
        """{name: (launches, total_ms)} -- call after torch.cuda.synchronize()."""
        return {k: (len(v), sum(s.elapsed_time(e) for s, e in v))
                for k, v in self.events.items()}

    def work(self):
        """{name: summed work of the launches whose wrapper reported it}."""
        return dict(self.amounts)


_timer: Optional[LaunchTimer] = None
_fns = {}


def set_timer(timer: Optional[LaunchTimer]) -> Optional[LaunchTimer]:
    """Install (or with None remove) the launch timer; returns the old one."""
    global _timer
    old, _timer = _timer, timer
    return old


def call(name: str, *args, work=None) -> None:
    """Call an entry point and raise RuntimeError on a non-zero status.
    ``work`` (optional) is the launch's algorithmic work for a LaunchTimer."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load(), name)
    if _timer is not None and _timer.wants(name):
        start, end = _timer.record(name, work)
        start.record()
        status = fn(*args)
        end.record()
    else:
        status = fn(*args)
    if status != 0:
        raise RuntimeError(
            f"{name} failed with {STATUS.get(status, status)}"
        )


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    """Raw device address of a tensor (None -> NULL)."""
    if t is None:
        return None
    return t.data_ptr()


_raw_stream = torch._C._cuda_getCurrentRawStream


def stream_handle(device: Optional[torch.device] = None) -> int:
    """hipStream_t of torch's current stream on `device` (read without
    building a torch Stream object)."""
    idx = device.index if device is not None else None
    return _raw_stream(torch.cuda.current_device() if idx is None else idx)


def require_device(*tensors: torch.Tensor) -> None:
    """The kernels only run on a ROCm device: refuse CPU tensors loudly."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "mlcg_amd kernels run on a ROCm GPU only; got a tensor on "
                f"{t.device}. Move the data and the model to 'cuda'."
            )


def version() -> str:
    return load().mlcg_version().decode()
