"""ctypes bindings of `libnca_hip.so` (the C ABI declared in include/nca_hip.h).

The library is loaded from the package directory. There is no fallback: when it is missing or
cannot be loaded every operator raises, so a silent CPU path can never stand in for the HIP one.
"""

from __future__ import annotations

import ctypes
import os

import torch

_SO = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnca_hip.so")

NCA_OK, NCA_ERR_INVALID, NCA_ERR_UNSUPPORTED, NCA_ERR_HIP = 0, 1, 2, 3
NOALLOC_SCRATCH_BYTES = 128 << 20  # NCA_NOALLOC_SCRATCH_BYTES of include/nca_hip.h
ADAMW_WORKSPACE_BYTES = 1024  # NCA_ADAMW_WORKSPACE_BYTES
PADDING = {"zero": 0, "wall": 1, "wrap": 2}
HEAD = {"mlp": 0, "l2": 1}
PRECISION = {"fp32": 0, "bf16": 1}
DAMAGE_GEOMETRY = {"ours": 0, "official": 1}

EXPORTS = (
    "nca_packed_weights_bytes",
    "nca_pack_weights",
    "nca_rollout",
    "nca_rollout_ws",
    "nca_rollout_workspace_bytes",
    "nca_step",
    "nca_fire_mask",
    "nca_readout",
    "nca_conf_select",
    "nca_last_error",
    "nca_version",
    "nca_set_kernel_path",
    "nca_set_window_steps",
    "nca_bptt_workspace_bytes",
    "nca_bptt_forward",
    "nca_bptt_forward_ws",
    "nca_bptt_backward",
    "nca_step_backward_workspace_bytes",
    "nca_step_backward",
    "nca_rollout_noalloc",
    "nca_prune_select",
    "nca_prune_select_rows",
    "nca_maze_metrics",
    "nca_sudoku_valid",
    "nca_adamw_ema",
    "nca_bptt_forward_pieces",
    "nca_set_piece_debug",
    "nca_set_bptt_backward_path",
    "nca_damage_clamp",
    "nca_pool_rows",
    "nca_init_state",
    "nca_maze_boards",
    "nca_sudoku_boards",
)


class CellDesc(ctypes.Structure):
    _fields_ = [
        ("channels", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("c_in", ctypes.c_int32),
        ("in_offset", ctypes.c_int32),
        ("c_out", ctypes.c_int32),
        ("out_offset", ctypes.c_int32),
        ("n_out", ctypes.c_int32),
        ("padding", ctypes.c_int32),
        ("head_kind", ctypes.c_int32),
        ("precision", ctypes.c_int32),
    ]


class CellWeights(ctypes.Structure):
    _fields_ = [
        ("kernels", ctypes.c_void_p),
        ("w1", ctypes.c_void_p),
        ("b1", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("b2", ctypes.c_void_p),
        ("head_w", ctypes.c_void_p),
        ("head_b", ctypes.c_void_p),
        ("pad_vec", ctypes.c_void_p),
    ]


class FireDesc(ctypes.Structure):
    _fields_ = [
        ("seed", ctypes.c_uint64),
        ("step_seeds", ctypes.c_void_p),
        ("fire_in", ctypes.c_void_p),
        ("row0", ctypes.c_int64),
        ("step0", ctypes.c_int64),
        ("p_fire", ctypes.c_float),
        ("p_low", ctypes.c_float),
        ("tau", ctypes.c_float),
        ("adaptive", ctypes.c_int32),
        ("given_confident", ctypes.c_int32),
    ]


class CellGrads(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("kernels", "w1", "b1", "w2", "b2", "head_w", "head_b")] + [
        ("accumulate", ctypes.c_int32)]


class AdamWDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_double) for n in ("lr", "beta1", "beta2", "eps", "weight_decay",
                                                "ema_decay", "max_norm")]


class PoolRowCopy(ctypes.Structure):
    _fields_ = [
        ("src", ctypes.c_void_p),
        ("dst", ctypes.c_void_p),
        ("src_row", ctypes.c_void_p),
        ("dst_row", ctypes.c_void_p),
        ("row_bytes", ctypes.c_int64),
        ("mode", ctypes.c_int32),
    ]


class BpttLoss(ctypes.Structure):
    _fields_ = [("targets", ctypes.c_void_p), ("loss_mask", ctypes.c_void_p),
                ("step_weights", ctypes.c_void_p)]


_lib = None


def library_path() -> str:
    return _SO


def load():
    """Load the HIP library (raises RuntimeError when it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_SO):
        raise RuntimeError(
            f"{_SO} is not built: run `python -m ncas_amd.build` (or __graft_entry__.build())"
        )
    L = ctypes.CDLL(_SO)
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    L.nca_packed_weights_bytes.argtypes = [ctypes.POINTER(CellDesc)]
    L.nca_packed_weights_bytes.restype = ctypes.c_size_t
    L.nca_pack_weights.argtypes = [ctypes.POINTER(CellDesc), ctypes.POINTER(CellWeights), vp, vp]
    L.nca_rollout.argtypes = [
        ctypes.POINTER(CellDesc), vp, i64, i32, i32, vp, vp, vp, vp, ctypes.POINTER(FireDesc),
        i32, vp, vp, vp, vp,
    ]
    L.nca_rollout_ws.argtypes = [
        ctypes.POINTER(CellDesc), vp, i64, i32, i32, vp, vp, vp, vp, ctypes.POINTER(FireDesc),
        i32, vp, vp, vp, vp, ctypes.c_size_t, vp,
    ]
    L.nca_rollout_noalloc.argtypes = [
        ctypes.POINTER(CellDesc), vp, i64, i32, i32, vp, vp, vp, vp, ctypes.POINTER(FireDesc),
        i32, vp, vp, vp, vp,
    ]
    L.nca_rollout_workspace_bytes.argtypes = [ctypes.POINTER(CellDesc), i64, i32, i32]
    L.nca_rollout_workspace_bytes.restype = ctypes.c_size_t
    L.nca_step.argtypes = [ctypes.POINTER(CellDesc), vp, i64, i32, i32, vp, vp, vp, vp, vp, vp, vp]
    L.nca_fire_mask.argtypes = [i64, i32, i32, ctypes.POINTER(FireDesc), i64, vp, vp, vp, vp]
    L.nca_readout.argtypes = [ctypes.POINTER(CellDesc), vp, i64, i32, i32, vp, vp, vp, vp, vp]
    L.nca_conf_select.argtypes = [vp, vp, i32, i32, i32, vp, vp]
    L.nca_bptt_workspace_bytes.argtypes = [ctypes.POINTER(CellDesc), i64, i32, i32, i32]
    L.nca_bptt_workspace_bytes.restype = ctypes.c_size_t
    L.nca_bptt_forward.argtypes = [ctypes.POINTER(CellDesc), vp, i64, i32, i32, vp, vp, vp,
                                   ctypes.POINTER(FireDesc), i32, vp, vp]
    L.nca_bptt_forward_ws.argtypes = [ctypes.POINTER(CellDesc), vp, i64, i32, i32, vp, vp, vp,
                                      ctypes.POINTER(FireDesc), i32, vp, vp, ctypes.c_size_t, vp]
    L.nca_bptt_backward.argtypes = [
        ctypes.POINTER(CellDesc), vp, ctypes.POINTER(CellWeights), i64, i32, i32, vp, vp,
        ctypes.POINTER(FireDesc), i32, ctypes.POINTER(BpttLoss), vp, ctypes.POINTER(CellGrads), vp,
        vp, vp, ctypes.c_size_t, vp,
    ]
    L.nca_step_backward_workspace_bytes.argtypes = [ctypes.POINTER(CellDesc), i64, i32, i32]
    L.nca_step_backward_workspace_bytes.restype = ctypes.c_size_t
    L.nca_step_backward.argtypes = [
        ctypes.POINTER(CellDesc), vp, ctypes.POINTER(CellWeights), i64, i32, i32, vp, vp, vp, vp,
        ctypes.POINTER(CellGrads), vp, vp, ctypes.c_size_t, vp,
    ]
    L.nca_prune_select.argtypes = [vp, vp, vp, i32, i32, i32, i32, ctypes.c_uint64, i64, vp, vp]
    L.nca_prune_select_rows.argtypes = [vp, vp, vp, i64, i32, i32, i32, i32, ctypes.c_uint64,
                                        i64, vp, vp]
    L.nca_maze_metrics.argtypes = [vp, vp, vp, vp, i64, i32, i32, i32, i64, i64, i64, vp, vp, vp]
    L.nca_sudoku_valid.argtypes = [vp, vp, vp, i64, i32, vp, vp]
    L.nca_adamw_ema.argtypes = [vp, vp, vp, vp, vp, i64, ctypes.POINTER(AdamWDesc), vp, vp, vp,
                                vp]
    L.nca_damage_clamp.argtypes = [vp, i64, i32, i32, i32, vp, i32, i32, ctypes.c_float, vp, vp,
                                   i32, i32, vp]
    L.nca_pool_rows.argtypes = [ctypes.POINTER(PoolRowCopy), i32, i64, vp]
    L.nca_init_state.argtypes = [vp, vp, vp, vp, i32, i64, i32, i32, i32, i32, i32, ctypes.c_float, vp, vp, vp]
    L.nca_maze_boards.argtypes = [i64, i32, ctypes.c_uint64, ctypes.c_double, i32, i32, vp, vp, vp,
                                  vp, i32]
    L.nca_sudoku_boards.argtypes = [i64, ctypes.c_uint64, i32, i32, vp, vp, vp, i32]
    L.nca_bptt_forward_pieces.argtypes = [ctypes.POINTER(CellDesc), i64, i32, i32, i32]
    L.nca_set_piece_debug.argtypes = [i32, i32, i32]
    L.nca_set_bptt_backward_path.argtypes = [i32]
    L.nca_last_error.restype = ctypes.c_char_p
    L.nca_version.restype = ctypes.c_int
    L.nca_set_kernel_path.argtypes = [ctypes.c_int]
    L.nca_set_window_steps.argtypes = [ctypes.c_int]
    for name in EXPORTS:
        getattr(L, name).restype = getattr(L, name).restype or ctypes.c_int
    _lib = L
    return L


def check(rc: int, what: str) -> None:
    if rc == NCA_OK:
        return
    msg = load().nca_last_error().decode(errors="replace")
    if rc in (NCA_ERR_INVALID, NCA_ERR_UNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def upload(a, device: torch.device) -> torch.Tensor:
    """A host array on the device through a fresh pinned buffer, without waiting: a copy from
    pageable memory would first wait for all the stream's queued work (torch keeps the pinned
    buffer alive until its copy has run). A CPU device gets a plain tensor."""
    t = torch.as_tensor(a)
    if torch.device(device).type != "cuda":
        return t.to(device)
    return t.pin_memory().to(device, non_blocking=True)


_COPY_STREAMS: dict = {}
_BESIDE_MIN_BYTES = 64 << 10


def upload_beside(a, device: torch.device) -> torch.Tensor:
    """`upload` on a stream of its own (default priority), for host arrays large enough that the
    runtime copies them with the DMA engine, which takes no compute unit: the copy starts when the
    host issues it, usually while the calling stream is still running earlier kernels, and the
    calling stream waits for it with an event instead of queueing its whole latency (about 25 us
    for a training batch's fresh boards). The memory comes from the copy stream's pool and is
    marked in use by the calling stream."""
    t = torch.as_tensor(a)
    device = torch.device(device)
    if device.type != "cuda" or t.numel() * t.element_size() < _BESIDE_MIN_BYTES:
        # small copies run as a kernel, which would take a compute unit from the calling
        # stream's kernels: those stay in stream order
        return upload(t, device)
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    side = _COPY_STREAMS.get(device.index)
    if side is None:
        side = _COPY_STREAMS[device.index] = torch.cuda.Stream(device)
    main = torch.cuda.current_stream(device)
    with torch.cuda.stream(side):
        d = t.pin_memory().to(device, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(side)
    main.wait_event(ev)
    d.record_stream(main)
    return d


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must be on the same GPU: the HIP path has no CPU fallback."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(
                f"the HIP operators need GPU tensors (got a tensor on {t.device}); "
                "there is no CPU implementation"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor given")
    return dev
