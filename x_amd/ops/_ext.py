"""Loader of the HIP library (libatl_hip.so) behind the atl ops API.

Replaces the reference's JIT-built pybind module (atl/ops/_ext.py:16-50, csrc/atl_cpu.cpp:299-329) with a
ctypes binding of the C-ABI declared in include/atl_hip.h.  ``get_ext()`` returns an object with the same
method names, argument order and return values as the pybind module (plus ``with_cuda = True``), so
atl/ops/functional.py-style callers work unchanged.  The HIP library handles device tensors only:

* device tensors always go to the HIP kernels; if the library is missing, ``get_ext()`` raises (no silent
  fallback);
* CPU tensors are not supported by the library (``ext_supports`` is False for them) and the ops use the
  pure-torch semantics in :mod:`x_amd.ops.reference`, as the reference does without its extension.

The library is built in-tree by ``python x_amd/csrc/build.py`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("ATL_HIP_LIB", Path(__file__).resolve().parents[1] / "csrc" / "libatl_hip.so"))

_P = ctypes.c_void_p
_I = ctypes.c_int64
_D = ctypes.c_double
_C = ctypes.c_int

# name -> argtypes (all return int status unless listed in _RESTYPE)
_SIGS = {
    "atl_splat_bilinear_fwd": [_P, _P, _P, _I, _I, _I, _I, _P, _P],
    "atl_splat_bilinear_bwd": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P],
    "atl_splat_gauss_fwd": [_P, _P, _P, _I, _I, _I, _I, _D, _I, _P, _P],
    "atl_splat_gauss_bwd": [_P, _P, _P, _P, _I, _I, _I, _I, _D, _I, _P, _P, _P],
    "atl_gather_bilinear_fwd": [_P, _P, _P, _I, _I, _I, _I, _P, _P],
    "atl_gather_bilinear_bwd": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P],
    "atl_voxel_grid": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P],
    "atl_sample_grid_fwd": [_P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _P, _P],
    "atl_sample_grid_bwd": [_P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _P, _P],
    "atl_sample_grid_bwd_pos": [_P, _P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _P, _P],
    "atl_field_channels_last": [_P, _I, _I, _I, _I, _P, _P],
    "atl_traj_displacement": [_P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _I, _P, _P],
    "atl_traj_visible": [_P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _I, _D, _I, _I, _P, _P, _I, _D, _I, _I, _P, _P],
    "atl_traj_origin": [_P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _I, _D, _I, _I, _P, _I, _P, _P],
    "atl_traj_origin_bwd": [_P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _I, _I, _P, _P, _P, _P],
    "atl_traj_field_bwd_planned": [_P, _P, _I, _I, _I, _I, _I, _P, _P, _P],
    "atl_traj_field_bwd_bytes": [_I, _I, _I, _I, _I],
    "atl_sample_grid_bwd_rows_bytes": [_I, _I, _I, _I, _I],
    "atl_plan_sort_bytes": [_I, _I, _I],
    "atl_plan_sort": [_P, _P, _P, _P, _I, _I, _D, _D, _D, _D, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _P],
    "atl_sample_grid_bwd_rows": [_P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _P, _P, _I, _P],
    "atl_traj_field_bwd": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _I, _P, _P],
    "atl_traj_pos_bwd_cl": [_P, _P, _I, _P, _I, _I, _I, _P, _P, _I, _P, _P],
    "atl_traj_gout": [_P, _P, _I, _I, _I, _P, _P],
    "atl_sample_grid_fwd_cl": [_P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _P, _P],
    "atl_sample_grid_bwd_pos_cl": [_P, _P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _P, _P],
    "atl_event_noise": [_P, _I, ctypes.c_uint64, ctypes.c_uint64, _D, _C, _P, _P, _P],
    "atl_image_variance_ws_bytes": [_I, _I],
    "atl_image_variance": [_P, _I, _I, _P, _P, _P, _I, _P],
    "atl_image_variance_bwd": [_P, _P, _P, _I, _I, _P, _P],
    "atl_plan_stats": [_P, _I, _P, _I, _P, _P],
    "atl_plan_count": [_P, _P, _P, _P, _I, _I, _D, _D, _D, _D, _I, _I, _I, _P, _P],
    "atl_scan_counts": [_P, _I, _P, _P, _P],
    "atl_scan_work_size": [_I],
    "atl_fill_i32": [_P, _I, _C, _P],
    "atl_plan_fill": [_P, _P, _P, _P, _I, _I, _D, _D, _D, _D, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P],
    "atl_plan_anchors": [_P, _P, _P, _P, _P, _I, _I, _D, _D, _D, _I, _I, _I, _P, _P, _P, _P, _P],
    "atl_ats_pair_fwd": [_P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _I, _P, _I, _I, _I, _D, _D, _D, _P, _P, _P],
    "atl_ats_pair_bwd": [_P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _I, _P, _I, _I, _I, _D, _D, _D, _I, _P,
                         _P],
    "atl_ats_pair_ws_bytes": [_I, _I, _I, _I],
    "atl_ats_pair_bwd_ws_bytes": [_I, _I, _I, _I, _I, _I],
    "atl_ats_pair_fwd_ws": [_P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _I, _P, _I, _I, _I, _D, _D, _D, _P, _P, _P,
                            _I, _P],
    "atl_ats_pair_bwd_ws": [_P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _I, _P, _I, _I, _I, _D, _D, _D, _I,
                            _P, _P, _I, _P],
    "atl_ats_pair_bwd_ws_binned": [_P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _I, _P, _I, _I, _I, _D, _D, _D, _I,
                            _P, _P, _I, _P],
    "atl_window_counts": [_P, _P, _I, _P, _I, _D, _P, _P],
    "atl_check_sorted": [_P, _P, _I, _P, _P],
    "atl_bin_counts": [_P, _P, _I, _I, _I, _P, _P],
    "atl_bin_counts_sorted": [_P, _P, _I, _I, _I, _P, _P],
    "atl_visible_fraction": [_P, _P, _P, _P, _I, _P, _P, _I, _I, _D, _I, _I, _P, _P],
    "atl_flow_interleave": [_P, _I, _I, _I, _P, _P],
    "atl_sample_flow_il": [_P, _I, _I, _I, _P, _P, _I, _I, _I, _P, _P],
    "atl_anchored_epilogue_fwd": [_P, _P, _P, _I, _D, _D, _P, _P, _P, _P],
    "atl_anchored_epilogue_bwd": [_P, _P, _P, _I, _P, _P],
    "atl_anchored_score_mean_scratch_bytes": [],
    "atl_anchored_score_mean_fwd": [_P, _P, _P, _I, _D, _D, _P, _P, _P, _P, _P],
    "atl_anchored_score_mean_bwd": [_P, _P, _P, _I, _P, _P],
    "atl_grid_plan_bytes": [_I, _I, _I, _I],
    "atl_tile_ws_bytes": [_I, _I, _I, _I],
    "atl_splat_gauss_ws_bytes": [_I, _I, _I, _I, _I],
    "atl_splat_gauss_fwd_ws": [_P, _P, _P, _I, _I, _I, _I, _D, _I, _P, _P, _I, _P],
    "atl_splat_bilinear_fwd_ws": [_P, _P, _P, _I, _I, _I, _I, _P, _P, _I, _P],
    "atl_splat_bilinear_fwd_noalloc": [_P, _P, _P, _I, _I, _I, _I, _P, _P],
    "atl_init": [],
    "atl_gather_bilinear_bwd_ws": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _I, _P],
    "atl_grid_plan": [_I, _I, _I, _P, _P, _I, _I, _I, _P, _I, _P],
    "atl_sample_grid_bwd_planned": [_P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _P, _P],
    "atl_sample_grid_bwd_binned": [_P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _P, _P, _I, _P],
    "atl_fast_geometry_init": [_I, _I, _I, _I, _I, _I, _D, _D, _D, _P],
    "atl_fast_plan": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P],
    "atl_fast_pair_fwd": [_P, _P, _P, _P, _P],
    "atl_fast_pair_bwd": [_P, _P, _P, _P, _P],
    "atl_fast_plan_traj": [_P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _P],
    "atl_fast_pair_bwd_traj": [_P, _P, _P, _P, _I, _P, _P, _P, _P],
    "atl_knn_ws_bytes": [_I, _I],
    "atl_voxel_ws_bytes": [_I, _I, _I, _I, _I],
    "atl_voxel_grid_ws": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _I, _P],
    "atl_knn_indices": [_P, _I, _P, _I, _I, _I, _P, _P, _I, _P],
    "atl_fast_pair_bwd_flow": [_P, _P, _P, _I, _I, _I, _I, _P, _P],
    "atl_fast_pair_bwd_src": [_P, _P, _P, _P],
    "atl_fast_flow_adjoint": [_P, _P, _I, _I, _I, _I, _P, _P],
    "atl_warp_splat_gather_ws_bytes": [_I, _I, _I, _I, _I, _I],
    "atl_warp_splat_gather_fwd": [_P, _I, _I, _I, _P, _P, _P, _I, _I, _I, _D, _I, _P, _P, _P, _I, _P],
    "atl_warp_splat_gather_bwd": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _D, _P, _P, _I, _P],
}
_RESTYPE = {"atl_scan_work_size": ctypes.c_int64, "atl_grid_plan_bytes": ctypes.c_int64,
            "atl_tile_ws_bytes": ctypes.c_int64, "atl_splat_gauss_ws_bytes": ctypes.c_int64,
            "atl_anchored_score_mean_scratch_bytes": ctypes.c_int64, "atl_knn_ws_bytes": ctypes.c_int64,
            "atl_voxel_ws_bytes": ctypes.c_int64, "atl_warp_splat_gather_ws_bytes": ctypes.c_int64,
            "atl_ats_pair_ws_bytes": ctypes.c_int64, "atl_ats_pair_bwd_ws_bytes": ctypes.c_int64, "atl_traj_field_bwd_bytes": ctypes.c_int64,
            "atl_sample_grid_bwd_rows_bytes": ctypes.c_int64, "atl_plan_sort_bytes": ctypes.c_int64,
            "atl_image_variance_ws_bytes": ctypes.c_int64,
"atl_last_error": ctypes.c_char_p, "atl_abi_version": ctypes.c_int}

class FastGeometry(ctypes.Structure):
    """Mirror of ``atl_fast_geometry`` (include/atl_hip.h): sizes, grid and workspace layout of the fused
    pair-sum path, filled by ``atl_fast_geometry_init``."""
    _fields_ = ([("version", ctypes.c_int32), ("bucket_shift", ctypes.c_int32)] +
                [(n, ctypes.c_int64) for n in ("N", "M", "B", "H", "W", "S")] +
                [(n, ctypes.c_double) for n in ("h", "tau", "cut")] +
                [(n, ctypes.c_float) for n in ("gx0", "gy0", "gx1", "gy1", "cell", "reserved_f")] +
                [(n, ctypes.c_int64) for n in ("GW", "GH", "ncell", "ncell_pad", "max_span", "ecap", "ws_bytes",
                                               "off_params", "off_cnt", "off_boff", "off_part", "off_start",
                                               "off_trec", "off_epos", "off_etim", "off_eself", "off_arec", "off_srec", "off_brec",
                                               "off_self")])


_LIB = None


class HipLibraryError(RuntimeError):
    """The HIP library is missing, or one of its entry points rejected its arguments."""


def load_library():
    """ctypes handle of libatl_hip.so (raises HipLibraryError if it is not built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise HipLibraryError(f"{LIB_PATH} is not built: run `python x_amd/csrc/build.py` "
                              "(x_amd runs device tensors on its HIP kernels only)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, args in _SIGS.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    for name, rt in _RESTYPE.items():
        getattr(lib, name).restype = rt
    lib.atl_last_error.argtypes = []
    if torch.cuda.is_available() and lib.atl_init() != 0:     # per-device set-up, before any graph capture
        raise HipLibraryError(lib.atl_last_error().decode())
    _LIB = lib
    return lib


def exported_symbols():
    return sorted(_SIGS) + ["atl_last_error", "atl_abi_version"]


_TIMED = {}          # entry point -> list of (start, end, events) per timed call, while kernel timing is on
_EVERY = {"n": 1, "calls": {}}   # time one call in n of each entry point
# position of the event count N in the arguments of the entry points whose calls are sized by it
_NARG = {"atl_sample_grid_fwd": 7, "atl_sample_grid_bwd_planned": 6, "atl_sample_grid_bwd_binned": 7, "atl_sample_grid_bwd_pos": 8,
         "atl_sample_grid_fwd_cl": 7, "atl_sample_flow_il": 6, "atl_sample_grid_bwd_pos_cl": 8, "atl_traj_displacement": 9,
         "atl_traj_gout": 2, "atl_traj_field_bwd_planned": 6, "atl_traj_field_bwd": 5, "atl_sample_grid_bwd_rows": 7, "atl_traj_origin": 9, "atl_traj_origin_bwd": 9, "atl_traj_pos_bwd_cl": 9,
         "atl_splat_gauss_fwd": 3, "atl_splat_gauss_bwd": 4, "atl_splat_gauss_fwd_ws": 3,
         "atl_gather_bilinear_fwd": 3, "atl_gather_bilinear_bwd_ws": 4, "atl_splat_bilinear_fwd_ws": 3,
         "atl_splat_bilinear_bwd": 4, "atl_voxel_grid_ws": 4, "atl_voxel_grid": 4,
         "atl_warp_splat_gather_fwd": 7, "atl_warp_splat_gather_bwd": 6}


def time_kernels(names, every: int = 1) -> dict:
    """Bracket later calls of the named entry points (the first call and then one in ``every``) with events on
    the caller's current stream (the stream the kernels run on); returns the live {name: [(start, end, events),
    ...]} record (events: the call's event count where the entry point has one, else None).  Each bracket
    holds the next launch back by a few microseconds, hence the sampling.  ``time_kernels(())`` turns timing
    off."""
    _TIMED.clear()
    _EVERY["n"], _EVERY["calls"] = max(int(every), 1), {}
    for n in names:
        _TIMED[n] = []
    return _TIMED


def timed_calls() -> dict:
    """Calls of each timed entry point since time_kernels (sampled or not)."""
    return dict(_EVERY["calls"])


def call(name: str, *args):
    """Invoke a C-ABI entry point; raise HipLibraryError with the library's message on failure."""
    lib = load_library()
    rec = _TIMED.get(name)
    if rec is not None:
        i = _EVERY["calls"].get(name, 0)
        _EVERY["calls"][name] = i + 1
        if i % _EVERY["n"]:
            rec = None
    if rec is not None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        rc = getattr(lib, name)(*args)
        e1.record()
        k = _NARG.get(name)
        rec.append((e0, e1, int(args[k]) if k is not None else None))
    else:
        rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.atl_last_error().decode(errors="replace")
        raise HipLibraryError(f"{name}: {msg}")
    return rc


def ptr(t: torch.Tensor | None):
    return ctypes.c_void_p(0) if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, dev: torch.device, shape=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device != dev:
        raise ValueError(f"{name} must be on {dev}, got {t.device}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None:
        for k, s in enumerate(shape):
            if s is not None and (t.dim() <= k or t.shape[k] != s):
                raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {shape}")
    return t


F32, I64 = torch.float32, torch.int64


class HipOps:
    """Same surface as the reference's extension module (csrc/atl_cpu.cpp:299-329), on HIP device tensors."""
    with_cuda = True

    # -------------------------------------------------------------------------------- splat / gather
    def splat_bilinear_fwd(self, pos, w, b, B, H, W):
        dev = pos.device
        N = pos.shape[0]
        _need(pos, "pos", F32, dev, (N, 2)); _need(w, "w", F32, dev, (N,)); _need(b, "b", I64, dev, (N,))
        img = torch.zeros(int(B), int(H), int(W), device=dev, dtype=F32)
        nbytes = load_library().atl_tile_ws_bytes(N, int(B), int(H), int(W)) if N > 0 and int(B) > 0 else -1
        with torch.cuda.device(dev):
            if nbytes >= 0:          # tile-binned LDS accumulation
                ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
                call("atl_splat_bilinear_fwd_ws", ptr(pos), ptr(w), ptr(b), N, int(B), int(H), int(W), ptr(img),
                     ptr(ws), nbytes, stream_of(pos))
            else:                    # too many tiles for the binning: one atomic per corner
                call("atl_splat_bilinear_fwd", ptr(pos), ptr(w), ptr(b), N, int(B), int(H), int(W), ptr(img),
                     stream_of(pos))
        return img

    def splat_bilinear_bwd(self, gimg, pos, w, b):
        dev = pos.device
        N = pos.shape[0]
        _need(gimg, "gimg", F32, dev); _need(pos, "pos", F32, dev, (N, 2)); _need(w, "w", F32, dev, (N,))
        _need(b, "b", I64, dev, (N,))
        B, H, W = gimg.shape
        gpos = torch.empty_like(pos); gw = torch.empty_like(w)
        with torch.cuda.device(dev):
            call("atl_splat_bilinear_bwd", ptr(gimg), ptr(pos), ptr(w), ptr(b), N, B, H, W, ptr(gpos), ptr(gw),
                 stream_of(pos))
        return [gpos, gw]

    def splat_gauss_fwd(self, pos, w, b, B, H, W, sigma, radius):
        dev = pos.device
        N = pos.shape[0]
        _need(pos, "pos", F32, dev, (N, 2)); _need(w, "w", F32, dev, (N,)); _need(b, "b", I64, dev, (N,))
        img = torch.zeros(int(B), int(H), int(W), device=dev, dtype=F32)
        nbytes = (load_library().atl_splat_gauss_ws_bytes(N, int(B), int(H), int(W), int(radius))
                  if N > 0 and int(B) > 0 else -1)
        with torch.cuda.device(dev):
            if nbytes >= 0:          # tile-binned LDS accumulation
                ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
                call("atl_splat_gauss_fwd_ws", ptr(pos), ptr(w), ptr(b), N, int(B), int(H), int(W), float(sigma),
                     int(radius), ptr(img), ptr(ws), nbytes, stream_of(pos))
            else:                    # radius beyond the tile engine's, or too many tiles: atomics per pixel
                call("atl_splat_gauss_fwd", ptr(pos), ptr(w), ptr(b), N, int(B), int(H), int(W), float(sigma),
                     int(radius), ptr(img), stream_of(pos))
        return img

    def splat_gauss_bwd(self, gimg, pos, w, b, sigma, radius):
        dev = pos.device
        N = pos.shape[0]
        _need(gimg, "gimg", F32, dev); _need(pos, "pos", F32, dev, (N, 2)); _need(w, "w", F32, dev, (N,))
        _need(b, "b", I64, dev, (N,))
        B, H, W = gimg.shape
        gpos = torch.empty_like(pos); gw = torch.empty_like(w)
        with torch.cuda.device(dev):
            call("atl_splat_gauss_bwd", ptr(gimg), ptr(pos), ptr(w), ptr(b), N, B, H, W, float(sigma), int(radius),
                 ptr(gpos), ptr(gw), stream_of(pos))
        return [gpos, gw]

    def gather_bilinear_fwd(self, img, pos, b):
        dev = pos.device
        N = pos.shape[0]
        _need(img, "img", F32, dev); _need(pos, "pos", F32, dev, (N, 2)); _need(b, "b", I64, dev, (N,))
        B, H, W = img.shape
        out = torch.empty(N, device=dev, dtype=F32)
        with torch.cuda.device(dev):
            call("atl_gather_bilinear_fwd", ptr(img), ptr(pos), ptr(b), N, B, H, W, ptr(out), stream_of(pos))
        return out

    def gather_bilinear_bwd(self, gval, img, pos, b):
        dev = pos.device
        N = pos.shape[0]
        _need(gval, "gval", F32, dev, (N,)); _need(img, "img", F32, dev); _need(pos, "pos", F32, dev, (N, 2))
        _need(b, "b", I64, dev, (N,))
        B, H, W = img.shape
        gimg = torch.zeros_like(img); gpos = torch.empty_like(pos)
        nbytes = load_library().atl_tile_ws_bytes(N, B, H, W) if N > 0 and B > 0 else -1
        with torch.cuda.device(dev):
            if nbytes >= 0:          # tile-binned LDS accumulation of gimg
                ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
                call("atl_gather_bilinear_bwd_ws", ptr(gval), ptr(img), ptr(pos), ptr(b), N, B, H, W, ptr(gimg),
                     ptr(gpos), ptr(ws), nbytes, stream_of(pos))
            else:
                call("atl_gather_bilinear_bwd", ptr(gval), ptr(img), ptr(pos), ptr(b), N, B, H, W, ptr(gimg),
                     ptr(gpos), stream_of(pos))
        return [gimg, gpos]

    def voxel_grid(self, pos, t, p, b, B, C, H, W):
        dev = pos.device
        N = pos.shape[0]
        _need(pos, "pos", F32, dev, (N, 2)); _need(t, "t", F32, dev, (N,)); _need(p, "p", F32, dev, (N,))
        _need(b, "b", I64, dev, (N,))
        vox = torch.zeros(int(B), int(C), int(H), int(W), device=dev, dtype=F32)
        nbytes = load_library().atl_voxel_ws_bytes(N, int(B), int(C), int(H), int(W)) if N > 0 and int(B) > 0 else -1
        with torch.cuda.device(dev):
            if nbytes >= 0:          # tile-binned LDS accumulation, the time bins as channels
                ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
                call("atl_voxel_grid_ws", ptr(pos), ptr(t), ptr(p), ptr(b), N, int(B), int(C), int(H), int(W),
                     ptr(vox), ptr(ws), nbytes, stream_of(pos))
            else:                    # too many tiles or bins for the LDS window: one atomic per corner
                call("atl_voxel_grid", ptr(pos), ptr(t), ptr(p), ptr(b), N, int(B), int(C), int(H), int(W),
                     ptr(vox), stream_of(pos))
        return vox

    # -------------------------------------------------------------------------------- pair sums
    def _pair_args(self, sy, sv, st, sid, cs, ax, at, ac, aid, sc):
        dev = ax.device
        E, M = st.shape[0], ax.shape[0]
        _need(sy, "src_y", F32, dev, (E, 2)); _need(sv, "src_v", F32, dev, (E, 2)); _need(st, "src_t", F32, dev)
        _need(sid, "src_id", I64, dev, (E,)); _need(cs, "cell_start", I64, dev)
        _need(ax, "anc_x", F32, dev, (M, 2)); _need(at, "anc_t", F32, dev, (M,)); _need(ac, "anc_cell", I64, dev,
                                                                                         (M, 3))
        _need(aid, "anc_id", I64, dev, (M,)); _need(sc, "slice_c", F32, dev)
        return E, M, cs.shape[0] - 1

    def _pair_ws(self, E, ncell, M, GW, dev, N=None, S=None):
        """Workspace of the pair entries; with the source count N and the slices S it also holds the backward's
        per-(source, slice) sums (the backward then adds no atomics)."""
        lib = load_library()
        nbytes = -1
        if N is not None and S is not None:
            nbytes = lib.atl_ats_pair_bwd_ws_bytes(E, ncell, M, int(GW), int(N), int(S))
        if nbytes < 0:
            nbytes = lib.atl_ats_pair_ws_bytes(E, ncell, M, int(GW))
        if nbytes < 0:
            raise HipLibraryError(f"ats_pair: no workspace size for E={E} ncell={ncell} M={M} GW={GW}")
        return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev), nbytes

    def ats_pair_fwd(self, sy, sv, st, sid, cs, ax, at, ac, aid, sc, S, GH, GW, h, tau, cut, count=None,
                     plan_order=False, keep_ws=False, n_src=None):
        """S (M,).  By default over a workspace allocated here with the output (atl_ats_pair_fwd_ws, anchors
        walked in cell order); ``plan_order`` selects the workspace-free entry.  ``keep_ws`` returns (S, ws):
        the workspace holds the binned anchors, which ats_pair_bwd(..., ws=ws) then reuses; with ``n_src`` (the
        backward's N) it is sized for the backward's per-(source, slice) sums too."""
        E, M, ncell = self._pair_args(sy, sv, st, sid, cs, ax, at, ac, aid, sc)
        out = torch.empty(M, device=ax.device, dtype=F32)
        args = (ptr(sy), ptr(sv), ptr(st), ptr(sid), ptr(cs), E, ncell, ptr(ax), ptr(at), ptr(ac), ptr(aid), M,
                ptr(sc), int(S), int(GH), int(GW), float(h), float(tau), float(cut), ptr(out), ptr(count))
        with torch.cuda.device(ax.device):
            if plan_order:
                call("atl_ats_pair_fwd", *args, stream_of(ax))
            else:
                ws, nbytes = self._pair_ws(E, ncell, M, GW, ax.device, n_src if keep_ws else None, S)
                call("atl_ats_pair_fwd_ws", *args, ptr(ws), nbytes, stream_of(ax))
                if keep_ws:
                    return out, ws
        return out

    def ats_pair_bwd(self, g, sy, sv, st, sid, cs, ax, at, ac, aid, sc, S, GH, GW, h, tau, cut, N,
                     per_pair_atomics=False, ws=None):
        """gv (N, 2).  By default the source-centric backward over a workspace allocated here with the output
        (atl_ats_pair_bwd_ws); ``per_pair_atomics`` selects the workspace-free entry (two atomics per pair);
        ``ws`` (from ats_pair_fwd(..., keep_ws=True) on the same plan) reuses the forward's anchor binning."""
        E, M, ncell = self._pair_args(sy, sv, st, sid, cs, ax, at, ac, aid, sc)
        _need(g, "gS", F32, ax.device, (M,))
        gv = torch.zeros(int(N), 2, device=ax.device, dtype=F32)
        args = (ptr(g), ptr(sy), ptr(sv), ptr(st), ptr(sid), ptr(cs), E, ncell, ptr(ax), ptr(at), ptr(ac), ptr(aid),
                M, ptr(sc), int(S), int(GH), int(GW), float(h), float(tau), float(cut), int(N), ptr(gv))
        with torch.cuda.device(ax.device):
            if per_pair_atomics:
                call("atl_ats_pair_bwd", *args, stream_of(ax))
            elif ws is not None:
                call("atl_ats_pair_bwd_ws_binned", *args, ptr(ws), ws.numel(), stream_of(ax))
            else:
                ws, nbytes = self._pair_ws(E, ncell, M, GW, ax.device, N, S)
                call("atl_ats_pair_bwd_ws", *args, ptr(ws), nbytes, stream_of(ax))
        return gv


_OPS = None


def get_ext() -> HipOps:
    """The HIP ops object (raises HipLibraryError if libatl_hip.so is not built)."""
    global _OPS
    if _OPS is None:
        load_library()
        _OPS = HipOps()
    return _OPS


def ext_supports(t: torch.Tensor) -> bool:
    """True for device tensors: they always run on the HIP library (which must then be built)."""
    return bool(t.is_cuda)
