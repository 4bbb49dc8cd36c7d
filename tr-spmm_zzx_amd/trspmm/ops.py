"""Device-level Python API over the C ABI: Format (builder output), Plan, spmm, sddmm.

Tensors handed to ``Plan.spmm`` / ``Plan.sddmm`` must already live on the GPU (fp16 operands,
float32 outputs); work is enqueued on the current torch stream.  Everything runs through
libtrspmm.so; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import hashlib
import os
from typing import Optional, Sequence, Union

import numpy as np
import torch

from . import _native as nat

# reference return-list names and element types (TR-source/Block/block_online.cpp:844-870)
SLOT_NAMES = [
    "t_rowkNew_offset", "t_blockNew_offset", "t_columnNew", "t_valueNew", "t_window_rowNew", "t_atomicNew",
    "t_binaryNew", "c_rowNew_offset", "c_rowNew", "c_atomicNew", "c_columnNew", "c_valueNew",
    "c_rowNew_offset_residue", "c_rowNew_residue", "c_atomicNew_residue", "c_columnNew_residue",
    "c_valueNew_residue", "s_columns", "s_masks", "s_values", "s_pos", "s_window", "s_offsets", "s_tile_window",
    "s_tile_group", "s_tile_columns", "s_packed_a", "s_packed_meta", "s_window_tile_offset",
    "spill_row", "spill_col", "spill_val",
]
SLOT_DTYPES = [np.int32, np.int32, np.int32, np.float32, np.int32, np.int32, np.int64,
               np.int32, np.int32, np.int32, np.int32, np.float32,
               np.int32, np.int32, np.int32, np.int32, np.float32,
               np.int32, np.uint8, np.float32, np.int8, np.int32, np.int32, np.int32, np.int32, np.int32,
               np.int32, np.int32, np.int32, np.int32, np.int32, np.float32]


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data if a.size else 0


class Format:
    """Output of the format builder (owns a C ``trs_format``)."""

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                nat.lib().trs_format_free(h)
            except (TypeError, AttributeError):   # interpreter shutdown: module globals already gone
                pass
            self._h = ctypes.c_void_p(0)

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def slot(self, i: int) -> np.ndarray:
        data = ctypes.c_void_p()
        n = ctypes.c_int64()
        nat.check(nat.lib().trs_format_slot(self._h, i, ctypes.byref(data), ctypes.byref(n)), "trs_format_slot")
        a = np.empty(n.value, dtype=SLOT_DTYPES[i])
        if n.value:
            ctypes.memmove(a.ctypes.data, data.value, n.value * a.itemsize)
        return a

    @property
    def window(self) -> int:
        return int(nat.lib().trs_format_window(self._h))

    @property
    def elapsed(self) -> float:
        return float(nat.lib().trs_format_elapsed(self._h))

    @property
    def canonical(self) -> bool:
        return bool(nat.lib().trs_format_canonical(self._h))

    def arrays(self) -> list:
        """The 29 reference arrays with the reference's shapes."""
        a = [self.slot(i) for i in range(29)]
        w = self.window
        g, t = a[21].shape[0], a[23].shape[0]
        a[17] = a[17].reshape(g, 4)
        a[18] = a[18].reshape(g, w)
        a[19] = a[19].reshape(g, w, 2)
        a[20] = a[20].reshape(g, w, 2)
        a[25] = a[25].reshape(t, 16)
        a[26] = a[26].reshape(t, 8, 4, 2)
        a[27] = a[27].reshape(t, 8)
        return a

    def spill(self) -> tuple:
        return self.slot(29), self.slot(30), self.slot(31)

    @property
    def rows(self) -> int:
        return int(nat.lib().trs_format_rows(self._h))

    def save(self, path) -> None:
        """Write the format to a cache file (trs_format_write: versioned, checksummed)."""
        nat.check(nat.lib().trs_format_write(self._h, os.fsencode(path)), "trs_format_write")

    @classmethod
    def load(cls, path) -> "Format":
        """Read a format written by :meth:`save`; raises TrsError for missing, truncated or
        corrupted files."""
        h = ctypes.c_void_p()
        nat.check(nat.lib().trs_format_read(os.fsencode(path), ctypes.byref(h)), "trs_format_read")
        return cls(h.value)

    def tensors(self) -> list:
        """The reference builder's return list: 29 CPU tensors + the build time as a float64
        scalar tensor (block_online.cpp:844-870)."""
        return [torch.from_numpy(a) for a in self.arrays()] + [torch.tensor(self.elapsed, dtype=torch.float64)]


_BUILD_DEFAULTS = dict(part_t=32, part_c=32, short_size=3, density=8, window=16, wide=16, tc_min_util=0.0,
                       sptc_min_util=0.5, sptc_threshold=12, skip_tc=None, unit_min_nnz=None, num_threads=0)


def build_format(rowptr, col, val, part_t: int = 32, part_c: int = 32, short_size: int = 3, density: int = 8,
                 window: int = 16, wide: int = 16, tc_min_util: float = 0.0, sptc_min_util: float = 0.5,
                 sptc_threshold: int = 12, skip_tc: Optional[bool] = None, unit_min_nnz: Optional[int] = None,
                 num_threads: int = 0) -> Format:
    """Run the builder (block_online.cpp:545-871 semantics).  ``skip_tc`` / ``unit_min_nnz`` of
    None read LIBRA_SKIP_TC / LIBRA_SPTC_UNIT_MIN_NNZ from the environment like the reference."""
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    col = np.ascontiguousarray(col, dtype=np.int32)
    val = np.ascontiguousarray(val, dtype=np.float32)
    p = nat.BuildParams()
    nat.lib().trs_build_params_default(ctypes.byref(p))
    p.part_size_t, p.part_size_c, p.short_size, p.density = part_t, part_c, short_size, density
    p.window, p.wide, p.tc_min_util, p.sptc_min_util = window, wide, tc_min_util, sptc_min_util
    p.sptc_threshold = sptc_threshold
    p.skip_tc = -1 if skip_tc is None else int(bool(skip_tc))
    p.sptc_unit_min_nnz = -1 if unit_min_nnz is None else int(unit_min_nnz)
    p.num_threads = num_threads
    h = ctypes.c_void_p()
    nat.check(nat.lib().trs_build_online(_ptr(rowptr), _ptr(col), _ptr(val), rowptr.shape[0] - 1, col.shape[0],
                                         ctypes.byref(p), ctypes.byref(h)), "trs_build_online")
    return Format(h.value)


class DeviceFormat:
    """Output of the GPU format builder (owns a C ``trs_dformat``): the same 32 slots as
    :class:`Format`, in device memory.  :meth:`download` returns the host :class:`Format`."""

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                nat.lib().trs_dformat_free(h)
            except (TypeError, AttributeError):
                pass
            self._h = ctypes.c_void_p(0)

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    @property
    def elapsed(self) -> float:
        return float(nat.lib().trs_dformat_elapsed(self._h))

    @property
    def rows(self) -> int:
        return int(nat.lib().trs_dformat_rows(self._h))

    @property
    def window(self) -> int:
        return int(nat.lib().trs_dformat_window(self._h))

    def slot_info(self, i: int) -> tuple:
        """(device pointer, element count) of slot i."""
        data = ctypes.c_void_p()
        n = ctypes.c_int64()
        nat.check(nat.lib().trs_dformat_slot(self._h, i, ctypes.byref(data), ctypes.byref(n)), "trs_dformat_slot")
        return data.value or 0, n.value

    def download(self) -> Format:
        h = ctypes.c_void_p()
        nat.check(nat.lib().trs_dformat_download(self._h, ctypes.byref(h)), "trs_dformat_download")
        return Format(h.value)


def build_format_device(rowptr: torch.Tensor, col: torch.Tensor, val: torch.Tensor, part_t: int = 32,
                        part_c: int = 32, short_size: int = 3, density: int = 8, window: int = 16,
                        wide: int = 16, tc_min_util: float = 0.0, skip_tc: Optional[bool] = None,
                        unit_min_nnz: Optional[int] = None, stream=None) -> DeviceFormat:
    """The format builder on the GPU (trs_build_online_device): int32 rowptr / col and float32 val
    on the current device, canonical rows, window <= 16.  Bit-exact with :func:`build_format`."""
    for name, t, dt in (("rowptr", rowptr, torch.int32), ("col", col, torch.int32), ("val", val, torch.float32)):
        if not (t.is_cuda and t.dtype == dt and t.dim() == 1 and t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous 1-D {dt} tensor on the GPU")
        _on_current_device(name, t)
    if col.shape[0] != val.shape[0]:
        raise ValueError("col and val must have the same length")
    p = nat.BuildParams()
    nat.lib().trs_build_params_default(ctypes.byref(p))
    p.part_size_t, p.part_size_c, p.short_size, p.density = part_t, part_c, short_size, density
    p.window, p.wide, p.tc_min_util = window, wide, tc_min_util
    p.skip_tc = -1 if skip_tc is None else int(bool(skip_tc))
    p.sptc_unit_min_nnz = -1 if unit_min_nnz is None else int(unit_min_nnz)
    h = ctypes.c_void_p()
    nat.check(nat.lib().trs_build_online_device(rowptr.data_ptr(), col.data_ptr() if col.numel() else None,
                                                val.data_ptr() if val.numel() else None, rowptr.shape[0] - 1,
                                                col.shape[0], ctypes.byref(p), _stream_ptr(stream),
                                                ctypes.byref(h)), "trs_build_online_device")
    return DeviceFormat(h.value)


def _env_setting(name: str) -> str:
    v = os.environ.get(name)
    return "unset" if v is None else v


def format_cache_key(rowptr, col, val, **params) -> str:
    """Hex digest identifying a builder run: the CSR bytes, every parameter, and the environment
    settings the builder reads when a parameter is left to the environment."""
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    col = np.ascontiguousarray(col, dtype=np.int32)
    val = np.ascontiguousarray(val, dtype=np.float32)
    h = hashlib.sha256()
    for a in (rowptr, col, val):
        h.update(np.int64(a.shape[0]).tobytes())
        h.update(a.tobytes())
    full = dict(_BUILD_DEFAULTS, **params)
    full.pop("num_threads", None)             # does not change the output
    if full.get("skip_tc") is None:
        full["env_skip_tc"] = _env_setting("LIBRA_SKIP_TC")
    if full.get("unit_min_nnz") is None:
        full["env_unit_min_nnz"] = _env_setting("LIBRA_SPTC_UNIT_MIN_NNZ")
    h.update(repr(sorted(full.items())).encode())
    return h.hexdigest()


def build_format_cached(rowptr, col, val, cache_dir, **params) -> Format:
    """build_format with a file cache: a format built before for the same CSR, parameters and
    environment is read back instead of rebuilt (the returned Format's ``from_cache`` says which).
    A cache file that cannot be read is rebuilt and overwritten."""
    os.makedirs(cache_dir, exist_ok=True)
    path = os.path.join(cache_dir, "format-" + format_cache_key(rowptr, col, val, **params)[:40] + ".trsf")
    if os.path.exists(path):
        try:
            f = Format.load(path)
            f.from_cache = True
            return f
        except nat.TrsError:
            pass
    f = build_format(rowptr, col, val, **params)
    f.save(path)
    f.from_cache = False
    return f


def _options(mfma_tc: bool, mfma_sptc: bool, sptc_min_fill: float, task_nnz: int, **extra) -> nat.PlanOptions:
    o = nat.PlanOptions()
    nat.lib().trs_plan_options_default(ctypes.byref(o))
    o.mfma_tc, o.mfma_sptc, o.sptc_min_fill, o.task_nnz = int(mfma_tc), int(mfma_sptc), sptc_min_fill, task_nnz
    for k, v in extra.items():
        if v is not None:
            setattr(o, k, int(v))
    return o


def _launch_stream(stream):
    return stream if stream is not None else torch.cuda.current_stream()


def _stream_ptr(stream) -> int:
    return int(_launch_stream(stream).cuda_stream)


def _on_current_device(name: str, t: torch.Tensor) -> None:
    """Plans are bound to the device they were created on, which the C ABI requires to be the
    current one (TRS_EDEVICE otherwise); operands on another GPU are refused here."""
    _on_device(name, t, torch.cuda.current_device())


def _on_device(name: str, t: torch.Tensor, dev: int) -> None:
    if t.device.index != dev:
        raise ValueError(f"{name} is on {t.device}, not on the current device cuda:{dev}")


class Plan:
    """Device-resident execution plan (owns a C ``trs_plan``)."""

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)
        self._dims = None    # (m, n, nnz): a plan is immutable, so read once
        self._ws = {}        # ("spmm" | "sddmm", K) -> workspace bytes

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                nat.lib().trs_plan_free(h)
            except (TypeError, AttributeError):   # interpreter shutdown: module globals already gone
                pass
            self._h = ctypes.c_void_p(0)

    @classmethod
    def from_format(cls, fmt: Union[Format, "DeviceFormat"], m: int, n: int, mfma_tc: bool = True, mfma_sptc: bool = True,
                    sptc_min_fill: float = 0.25, task_nnz: int = 0, piece_nnz: Optional[int] = None,
                    feature_lanes: Optional[int] = None, streaming: Optional[int] = None,
                    window_row_cap: Optional[int] = None, xcd_run: Optional[int] = None,
                    stage: Optional[int] = None, occupancy: Optional[int] = None,
                    xcd_split: Optional[int] = None, host_lowering: bool = False,
                    sptc_sparse: bool = True, hot_rows: Optional[int] = None,
                    split_dispatch: Optional[int] = None) -> "Plan":
        """Plan over the builder output (all shares + spill); a :class:`DeviceFormat` is lowered
        where it lives (trs_plan_create_dformat: the plan equals that of its downloaded format).  Tuning options: see trs_plan_options
        in include/trspmm.h (None keeps the library default).  host_lowering=True builds the
        residual on the host even when the format holds its input CSR (the plan is the same);
        sptc_sparse=False runs 2:4 tiles on the dense MFMA with zero fill instead of the sparse one."""
        o = _options(mfma_tc, mfma_sptc, sptc_min_fill, task_nnz, piece_nnz=piece_nnz,
                     feature_lanes=feature_lanes, streaming=streaming, window_row_cap=window_row_cap,
                     xcd_run=xcd_run, stage=stage, occupancy=occupancy, xcd_split=xcd_split, hot_rows=hot_rows,
                     split_dispatch=split_dispatch)
        o.host_lowering = int(bool(host_lowering))
        o.sptc_sparse = int(bool(sptc_sparse))
        h = ctypes.c_void_p()
        fn = "trs_plan_create_dformat" if isinstance(fmt, DeviceFormat) else "trs_plan_create"
        nat.check(getattr(nat.lib(), fn)(fmt.handle, m, n, ctypes.byref(o), ctypes.byref(h)), fn)
        return cls(h.value)

    @classmethod
    def for_sddmm(cls, fmt: Union[Format, "DeviceFormat"], m: int, n: int, mfma_tc: bool = True, mfma_sptc: bool = True,
                  sptc_min_fill: float = 0.25, task_nnz: int = 0, piece_nnz: Optional[int] = None,
                  feature_lanes: Optional[int] = None, xcd_run: Optional[int] = None,
                  sddmm_unroll: Optional[int] = None, stage: Optional[int] = None,
                  streaming: Optional[int] = None, xcd_split: Optional[int] = None,
                  host_lowering: bool = False, hot_rows: Optional[int] = None,
                  split_dispatch: Optional[int] = None, occupancy: Optional[int] = None) -> "Plan":
        """SDDMM plan on the hybrid tiling (dense tiles on MFMA, rest as CSR dot products);
        ``sddmm`` outputs follow the input CSR order.  ``streaming`` bit 1 (default on) writes the
        residual outputs with non-temporal stores.  host_lowering=True builds the residual on the
        host even when the format holds its input CSR (the plan is the same).  A
        :class:`DeviceFormat` is lowered where it lives (trs_plan_create_sddmm_dformat)."""
        o = _options(mfma_tc, mfma_sptc, sptc_min_fill, task_nnz, piece_nnz=piece_nnz,
                     feature_lanes=feature_lanes, xcd_run=xcd_run, sddmm_unroll=sddmm_unroll, stage=stage,
                     streaming=streaming, xcd_split=xcd_split, hot_rows=hot_rows, split_dispatch=split_dispatch,
                     occupancy=occupancy)
        o.host_lowering = int(bool(host_lowering))
        h = ctypes.c_void_p()
        fn = "trs_plan_create_sddmm_dformat" if isinstance(fmt, DeviceFormat) else "trs_plan_create_sddmm"
        nat.check(getattr(nat.lib(), fn)(fmt.handle, m, n, ctypes.byref(o), ctypes.byref(h)), fn)
        return cls(h.value)

    @classmethod
    def from_csr(cls, rowptr, col, val_f16, m: int, n: int, task_nnz: int = 0, piece_nnz: Optional[int] = None,
                 feature_lanes: Optional[int] = None, streaming: Optional[int] = None,
                 xcd_run: Optional[int] = None, stage: Optional[int] = None,
                 occupancy: Optional[int] = None, xcd_split: Optional[int] = None,
                 hot_rows: Optional[int] = None) -> "Plan":
        rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
        col = np.ascontiguousarray(col, dtype=np.int32)
        val = np.ascontiguousarray(val_f16, dtype=np.float16).view(np.uint16)
        # trs_plan_create_csr reads rowptr[0..m] and col / val up to rowptr[m]: refuse short arrays here
        if m < 0 or rowptr.ndim != 1 or rowptr.shape[0] != m + 1:
            raise ValueError(f"rowptr must hold m + 1 = {m + 1} entries (got {rowptr.shape})")
        nnz = int(rowptr[-1])
        if col.shape[0] < nnz or val.shape[0] < nnz:
            raise ValueError(f"col and val must hold at least rowptr[-1] = {nnz} entries "
                             f"(got {col.shape[0]} and {val.shape[0]})")
        o = _options(False, False, 1.0, task_nnz, piece_nnz=piece_nnz, feature_lanes=feature_lanes,
                     streaming=streaming, xcd_run=xcd_run, stage=stage, occupancy=occupancy,
                     xcd_split=xcd_split, hot_rows=hot_rows)
        h = ctypes.c_void_p()
        nat.check(nat.lib().trs_plan_create_csr(_ptr(rowptr), _ptr(col), _ptr(val), m, n, ctypes.byref(o),
                                                ctypes.byref(h)), "trs_plan_create_csr")
        return cls(h.value)

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def stats(self) -> dict:
        s = nat.PlanStats()
        nat.check(nat.lib().trs_plan_stats_get(self._h, ctypes.byref(s), ctypes.sizeof(s)), "trs_plan_stats_get")
        return {k: int(getattr(s, k)) for k, _ in nat.PlanStats._fields_}

    def workspace_bytes(self, K: int) -> int:
        key = ("spmm", K)
        if key not in self._ws:
            self._ws[key] = int(nat.lib().trs_spmm_workspace_bytes(self._h, K))
        return self._ws[key]

    def _shape(self):
        if self._dims is None:
            st = self.stats()
            self._dims = (st["m"], st["n"], st["nnz"])
        return self._dims

    @staticmethod
    def _temporaries(stream, make):
        """Allocate the call's temporaries on the launch stream (entered only when something is
        allocated: the context switch costs more than the call's checks)."""
        with torch.cuda.stream(_launch_stream(stream)):
            return make()

    def spmm(self, B: torch.Tensor, out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
             stream=None) -> torch.Tensor:
        """C = A B for B [n, K] fp16 on the GPU; returns float32 [m, K].  Temporaries (a defaulted
        ``out`` or workspace) are allocated on the launch stream, so the caching allocator does not
        hand them to other work while the kernels on ``stream`` still use them."""
        m, n, _ = self._shape()
        if not (B.is_cuda and B.dtype == torch.float16 and B.dim() == 2 and B.shape[0] == n):
            raise ValueError(f"B must be a CUDA fp16 tensor of shape [{n}, K]")
        dev = torch.cuda.current_device()
        _on_device("B", B, dev)
        if B.stride(1) != 1:
            B = B.contiguous()
        K = B.shape[1]
        need = self.workspace_bytes(K)
        new_ws = need and (workspace is None or workspace.numel() * workspace.element_size() < need)
        if out is None or new_ws:
            out, workspace = self._temporaries(stream, lambda: (
                out if out is not None else torch.empty((m, K), dtype=torch.float32, device=B.device),
                torch.empty(need, dtype=torch.uint8, device=B.device) if new_ws else workspace))
        if not (out.is_cuda and out.dtype == torch.float32 and tuple(out.shape) == (m, K) and out.stride(1) == 1):
            raise ValueError("out must be a CUDA float32 tensor [m, K] with unit column stride")
        _on_device("out", out, dev)
        if need:
            if not (workspace.is_cuda and workspace.is_contiguous()):
                raise ValueError("workspace must be a contiguous CUDA tensor")
            _on_device("workspace", workspace, dev)
        ws_ptr = workspace.data_ptr() if need else 0
        nat.check(nat.lib().trs_spmm_f16(self._h, B.data_ptr(), B.stride(0), K, out.data_ptr(), out.stride(0),
                                         ws_ptr, need, _stream_ptr(stream)), "trs_spmm_f16")
        return out

    def sddmm_workspace_bytes(self, K: int) -> int:
        key = ("sddmm", K)
        if key not in self._ws:
            self._ws[key] = int(nat.lib().trs_sddmm_workspace_bytes(self._h, K))
        return self._ws[key]

    def sddmm(self, X: torch.Tensor, Y: torch.Tensor, out: Optional[torch.Tensor] = None,
              workspace: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """out[e] = X[row_e] . Y[col_e] for every stored entry (CSR order); float32 [nnz].  A given
        ``out`` must be a contiguous float32 CUDA tensor of at least ``stats()['nnz']`` elements.
        Plans with staged hot rows take a workspace (``sddmm_workspace_bytes(K)``), allocated on the
        launch stream when not given."""
        m, n, nnz = self._shape()
        dev = torch.cuda.current_device()
        for name, t, rows in (("X", X, m), ("Y", Y, n)):
            if not (t.is_cuda and t.dtype == torch.float16 and t.dim() == 2 and t.shape[0] == rows):
                raise ValueError(f"{name} must be a CUDA fp16 tensor with {rows} rows")
            _on_device(name, t, dev)
        if X.shape[1] != Y.shape[1]:
            raise ValueError("X and Y need the same feature width")
        X = X if X.stride(1) == 1 else X.contiguous()
        Y = Y if Y.stride(1) == 1 else Y.contiguous()
        K = X.shape[1]
        need = self.sddmm_workspace_bytes(K)
        new_ws = need and (workspace is None or workspace.numel() * workspace.element_size() < need)
        if out is None or new_ws:
            out, workspace = self._temporaries(stream, lambda: (
                out if out is not None else torch.empty(nnz, dtype=torch.float32, device=X.device),
                torch.empty(need, dtype=torch.uint8, device=X.device) if new_ws else workspace))
        if not (isinstance(out, torch.Tensor) and out.is_cuda and out.dtype == torch.float32 and out.is_contiguous()
                and out.numel() >= nnz):
            raise ValueError(f"out must be a contiguous CUDA float32 tensor of at least {nnz} elements")
        _on_device("out", out, dev)
        if need:
            if not (workspace.is_cuda and workspace.is_contiguous()):
                raise ValueError("workspace must be a contiguous CUDA tensor")
            _on_device("workspace", workspace, dev)
        nat.check(nat.lib().trs_sddmm_f16_ws(self._h, X.data_ptr(), X.stride(0), Y.data_ptr(), Y.stride(0), K,
                                             out.data_ptr(), workspace.data_ptr() if need else 0, need,
                                             _stream_ptr(stream)), "trs_sddmm_f16_ws")
        return out


def spmm(plan: Plan, B: torch.Tensor, **kw) -> torch.Tensor:
    return plan.spmm(B, **kw)


def sddmm(plan: Plan, X: torch.Tensor, Y: torch.Tensor, **kw) -> torch.Tensor:
    return plan.sddmm(X, Y, **kw)
