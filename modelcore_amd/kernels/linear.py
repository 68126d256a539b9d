"""Decode-sized products on the matrix cores: ``y = x . W^T`` for at most 64 rows of bf16
activations, the projection GEMMs of a decode step (``F.linear`` in the reference's
``Linear.forward``, modelcore/components/linear.py:13-14).

With 64 or fewer rows each weight byte is used at most 64 times, so the product is bound by
reading W once from HBM. ``mcamd_linear_bf16`` streams tiles of W (128 rows for wide products,
64 otherwise) and the activations through LDS with coalesced loads; when N has too few tiles to
fill the GPU the K range is split and the partial products are summed in a fixed order by a
second kernel (deterministic, fp32 accumulation). ``linear_bf16_partials`` leaves that sum to a
consumer that sums them itself (the fused residual and pre-attention steps), and
``linear_bf16_gated`` computes a gated MLP's ``silu(x W_gate^T) * (x W_up^T)`` from W_gate and
W_up interleaved in 64-row blocks. ``supported`` says which shapes they take.
"""
from __future__ import annotations

import torch

from modelcore_amd import _ext

__all__ = ["supported", "linear_bf16", "linear_bf16_partials", "Partials", "k_splits",
           "gated_supported", "interleave_gate_up", "linear_bf16_gated", "tile_weight",
           "untile_weight"]

MAX_ROWS = 64
TILE_N = 64     # rows of W per workgroup (four waves)
WIDE_N = 192 * 128  # from this N on, 128-row tiles of eight waves with no K split
STAGE_K = 128   # k per pipeline stage
_CUS = 256
_WS: dict = {}
_RETIRED: list = []  # outgrown workspaces, kept alive: a captured graph may still write to them


def supported(x: torch.Tensor, w: torch.Tensor) -> bool:
    """Whether ``linear_bf16(x, w)`` takes these operands (device, dtype, sizes, layout)."""
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or x.device.type != "cuda" \
            or w.device != x.device or w.dim() != 2 or not w.is_contiguous():
        return False
    n, k = w.shape
    if x.shape[-1] != k or n % TILE_N or k % STAGE_K or 128 * k * 2 >= 2 ** 31:
        return False
    rows = x.numel() // k if k else 0
    return 0 < rows <= MAX_ROWS


def k_splits(m: int, n: int, k: int) -> int:
    """The K split for an (m, n, k) product: 1 when N alone fills the GPU (the library then runs
    128-row tiles of eight waves), else the largest power of two that keeps the tiles x splits
    within one workgroup per CU -- 128-row tiles for more than 16 rows (the library then runs
    eight waves), 64-row tiles otherwise. Measured on MI355X with cold weights and 64 rows: 6144 x
    4096 at S = 4 with 128-row tiles 12.6 us against 14.4 at S = 2 with 64-row ones, 4096 x 14336
    at S = 8 22.8 against 25.1 at S = 4; the 64-row sampling step 0.5-1.5% faster overall (the
    residual and pre-attention steps sum twice the partials)."""
    if n >= WIDE_N:
        return 1
    # More than 16 rows: 128-row tiles of eight waves (half the activation traffic per weight
    # byte), split twice as often as 64-row tiles would be.
    tile = 2 * TILE_N if m > 16 and n % (2 * TILE_N) == 0 else TILE_N
    tiles = n // tile
    best = 1
    for s in (2, 4, 8, 16):
        if k % (STAGE_K * s) == 0 and tiles * s <= _CUS:
            best = s
    return best


def _workspace(device, nbytes):
    """The split-K partials buffer of this device, at least `nbytes` (None for 0).

    One buffer per device is shared by every call on that device's stream. A graph captured with
    it holds its address, so an outgrown buffer is retired but kept alive (never returned to the
    caching allocator, whose next tensor would otherwise receive the graph's writes). During
    capture a too-small buffer is not replaced: the call gets one of the graph's own pool."""
    if nbytes == 0:
        return None
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _WS.get(idx)
    if ws is not None and ws.numel() >= nbytes:
        return ws
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    size = max(nbytes, 2 * ws.numel() if ws is not None else 0, 1 << 20)
    if ws is not None:
        _RETIRED.append(ws)
    ws = _WS[idx] = torch.empty(size, dtype=torch.uint8, device=device)
    return ws


def linear_bf16(x: torch.Tensor, w: torch.Tensor, splits: int | None = None) -> torch.Tensor:
    """(..., k) bf16 x (n, k) bf16 -> (..., n) bf16, for at most 64 rows of x."""
    _ext.require_rocm(x, w, what="linear_bf16")
    if not supported(x, w):
        raise ValueError(f"linear_bf16 takes bf16 x with <= {MAX_ROWS} rows and a contiguous bf16 "
                         f"(n, k) weight, n % {TILE_N} == 0, k % {STAGE_K} == 0; got x "
                         f"{tuple(x.shape)} {x.dtype}, w {tuple(w.shape)} {w.dtype}")
    n, k = w.shape
    x2 = x.reshape(-1, k)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    s = splits if splits is not None else k_splits(m, n, k)
    lib = _ext.lib()
    need = lib.mcamd_linear_bf16_workspace_bytes(m, n, s)
    ws = _workspace(x.device, need)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)
    st = lib.mcamd_linear_bf16(x2.data_ptr(), x2.stride(0), w.data_ptr(), y.data_ptr(), n, m, n,
                               k, s, ws.data_ptr() if ws is not None else None,
                               ws.numel() if ws is not None else 0, _ext.stream_handle(x.device))
    _ext.check(st, "linear_bf16")
    return y.view(*x.shape[:-1], n)


class Partials:
    """The K-split partial products of x . W^T, unsummed: ``part`` is (splits, rows, n) fp32 and
    ``shape`` the shape the summed product would have. Only a consumer that sums them itself
    takes one (``kernels.residual.residual_rmsnorm``)."""
    __slots__ = ("part", "splits", "shape")

    def __init__(self, part: torch.Tensor, splits: int, shape: tuple):
        self.part, self.splits, self.shape = part, splits, shape


def linear_bf16_partials(x: torch.Tensor, w: torch.Tensor, splits: int | None = None) -> Partials:
    """``linear_bf16(x, w)`` with the sum of its K-split partials left to the consumer."""
    _ext.require_rocm(x, w, what="linear_bf16_partials")
    if not supported(x, w):
        raise ValueError(f"linear_bf16_partials takes what linear_bf16 takes; got x "
                         f"{tuple(x.shape)} {x.dtype}, w {tuple(w.shape)} {w.dtype}")
    n, k = w.shape
    x2 = x.reshape(-1, k)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    s = splits if splits is not None else k_splits(m, n, k)
    part = torch.empty(s, m, n, dtype=torch.float32, device=x.device)
    st = _ext.lib().mcamd_linear_bf16_partials(x2.data_ptr(), x2.stride(0), w.data_ptr(),
                                               part.data_ptr(), m, n, k, s,
                                               _ext.stream_handle(x.device))
    _ext.check(st, "linear_bf16_partials")
    return Partials(part, s, (*x.shape[:-1], n))


GATE_BLOCK = 64  # rows of W_gate, then of W_up, alternating in the interleaved gate/up weight


def interleave_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """[W_gate; W_up] with their rows interleaved in blocks of 64 (gate rows 64 b .. 64 b + 63,
    then the up rows of the same units): the layout linear_bf16_gated reads. (2 hidden, k)."""
    hid, k = w_gate.shape
    if w_up.shape != w_gate.shape or hid % GATE_BLOCK:
        raise ValueError(f"gate {tuple(w_gate.shape)} / up {tuple(w_up.shape)}: need equal shapes "
                         f"with a multiple of {GATE_BLOCK} rows")
    return torch.stack([w_gate.reshape(-1, GATE_BLOCK, k), w_up.reshape(-1, GATE_BLOCK, k)],
                       dim=1).reshape(2 * hid, k)


def split_gate_up(out: torch.Tensor):
    """gate, up (each (..., hidden), strided views) of x . W^T for an interleaved W."""
    n = out.shape[-1]
    blocks = out.view(*out.shape[:-1], n // (2 * GATE_BLOCK), 2, GATE_BLOCK)
    return blocks[..., 0, :], blocks[..., 1, :]


TILE_ROWS, TILE_K = 64, 128  # one block of a tiled weight: 64 rows x 128 columns, 16 KB


def tile_weight(w: torch.Tensor) -> torch.Tensor:
    """(n, k) -> (n / 64, k / 128, 64, 128) contiguous blocks: the layout in which the weight
    stream of the gated product reads whole 1 KB runs (a copy; untile_weight undoes it)."""
    n, k = w.shape
    if n % TILE_ROWS or k % TILE_K:
        raise ValueError(f"tiling needs n % {TILE_ROWS} == 0 and k % {TILE_K} == 0; got "
                         f"{tuple(w.shape)}")
    return w.reshape(n // TILE_ROWS, TILE_ROWS, k // TILE_K, TILE_K).transpose(1, 2).contiguous()


def untile_weight(wt: torch.Tensor) -> torch.Tensor:
    """The row-major (n, k) weight of a tile_weight result (a copy)."""
    g, s, r, c = wt.shape
    return wt.transpose(1, 2).reshape(g * r, s * c)


def gated_supported(x: torch.Tensor, w: torch.Tensor) -> bool:
    """Whether linear_bf16_gated(x, w) takes these operands (w row-major or tiled)."""
    if w.dim() != 4:
        return supported(x, w) and w.shape[0] % (2 * GATE_BLOCK) == 0
    if w.shape[2:] != (TILE_ROWS, TILE_K) or not w.is_contiguous():
        return False
    n, k = w.shape[0] * TILE_ROWS, w.shape[1] * TILE_K
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or x.device.type != "cuda" \
            or w.device != x.device:
        return False
    if x.shape[-1] != k or n % (2 * GATE_BLOCK) or 128 * k * 2 >= 2 ** 31:
        return False
    return 0 < x.numel() // k <= MAX_ROWS


def linear_bf16_gated(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """silu(x . W_gate^T) * (x . W_up^T), (..., hidden) bf16, for the interleaved W of
    interleave_gate_up, row-major or tiled (tile_weight); torch's rounding of the separate bf16
    ops."""
    _ext.require_rocm(x, w, what="linear_bf16_gated")
    if not gated_supported(x, w):
        raise ValueError(f"linear_bf16_gated takes what linear_bf16 takes, with 2 * 64 | n; got x "
                         f"{tuple(x.shape)} {x.dtype}, w {tuple(w.shape)} {w.dtype}")
    tiled = w.dim() == 4
    n, k = (w.shape[0] * TILE_ROWS, w.shape[1] * TILE_K) if tiled else w.shape
    hid = n // 2
    x2 = x.reshape(-1, k)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    h = torch.empty(m, hid, dtype=torch.bfloat16, device=x.device)
    st = _ext.lib().mcamd_linear_bf16_gated(x2.data_ptr(), x2.stride(0), w.data_ptr(),
                                            h.data_ptr(), hid, m, hid, k, _ext.ACT_SILU,
                                            int(tiled), _ext.stream_handle(x.device))
    _ext.check(st, "linear_bf16_gated")
    return h.view(*x.shape[:-1], hid)
