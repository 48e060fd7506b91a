"""sparsecore_amd.ops — spmm, its autograd Function and the transpose cache.

Drop-in for ``sparselab/ops.py``: same public ``spmm(W, X, *, kernel)``, same
``_SpMMFunction.apply(W_values, W, X, kernel)`` contract, same
``_transpose_cache`` / ``_cached_transpose`` / ``_clear_transpose_cache``
(cache entries are ``(topology_version, (nrows, ncols), WT, perm)``).

Every kernel runs on the HIP device through the C-ABI library:

    forward  Y  = W·X               slk_spmm                 (ops.py:144-165)
    backward dW = SDDMM(dY, X)      slk_sddmm                (ops.py:186-192)
             WT = cached transpose  slk_transpose_refresh on a hit,
                                    slk_transpose_count/fill on a miss (ops.py:70-99)
             dX = WT·dY             slk_spmm on WT           (ops.py:201-203)

Tensors on the CPU are rejected with RuntimeError (the reference rejected
non-CPU tensors the same way; this build is GPU-only and has no CPU path).
"""

from __future__ import annotations

import weakref

import torch

from . import _lib, layout
from .layout import PaddedCSR, transpose_with_perm, transposes_with_perm

__all__ = ["spmm", "dense_grad"]

_KERNELS = ("auto", "simd", "scalar")

# Key: id(W). Value: (topology_version, (nrows, ncols), WT, perm).
_transpose_cache: dict[int, tuple[int, tuple[int, int], PaddedCSR, torch.Tensor]] = {}


def _drop_entry(key: int) -> None:
    _transpose_cache.pop(key, None)


def _cached_transpose(W: PaddedCSR) -> PaddedCSR:
    """W's transpose, rebuilt only when W's topology changes (ops.py:70-99).

    Hit (same id, topology_version and shape): refresh the live WT values from
    W.values through perm on the device and return the same WT object.
    Miss: rebuild on the device and store the entry. Entries are dropped when
    W is garbage collected, so a recycled id() can never return a stale WT.
    """
    key = id(W)
    cur_version = W.topology_version
    cur_shape = (int(W.nrows), int(W.ncols))
    cached = _transpose_cache.get(key)
    if cached is not None and cached[0] == cur_version and cached[1] == cur_shape:
        _, _, WT, perm = cached
        _lib.transpose_refresh(W.values, perm, WT.values)
        return WT
    WT, perm = transpose_with_perm(W)
    if cached is None:
        weakref.finalize(W, _drop_entry, key)
    _transpose_cache[key] = (cur_version, cur_shape, WT, perm)
    return WT


def _rigl_update_cached(W: PaddedCSR, k_drop: int, dY: torch.Tensor, X: torch.Tensor) -> None:
    """``W._rigl_update(k_drop, dY, X)``, then W's cached transpose rebuilt for
    the new topology, as ``_cached_transpose`` would on its next call, with one
    host read for both: the rebuild is queued right behind the row rewrite,
    its slot arrays sized from the live slots before the update (rows only
    shrink), and its capacity read with the RigL counts. Without a cached
    transpose of W this is ``W._rigl_update``."""
    key = id(W)
    if key not in _transpose_cache:
        W._rigl_update(k_drop, dY, X)
        return
    staged = {}

    def then():
        staged["t"] = layout._transpose_queue(W, 0.2, W.nnz)
        return staged["t"]["counts"], finish

    def finish(host):
        if host is None:  # the exact path rewrote W after the queued rebuild
            _cached_transpose(W)
            return
        WT, perm = layout._transpose_take(W, staged["t"], host, W.nnz)
        _transpose_cache[key] = (W.topology_version, (int(W.nrows), int(W.ncols)), WT, perm)

    W._rigl_update(k_drop, dY, X, then=then)


def _cached_transpose_structure(W: PaddedCSR):
    """(WT, perm) from the transpose cache, rebuilt when W's topology changed
    (as ``_cached_transpose``) but without refreshing WT's values: for a
    caller that reads W's values through perm (slk_backward_fused). The next
    ``_cached_transpose`` refreshes them as on every hit."""
    key = id(W)
    cached = _transpose_cache.get(key)
    if cached is not None and cached[0] == W.topology_version and \
            cached[1] == (int(W.nrows), int(W.ncols)):
        return cached[2], cached[3]
    WT = _cached_transpose(W)
    return WT, _transpose_cache[key][3]


def _rebuild_stale_transposes(Ws) -> None:
    """Rebuilds, in one batch (one device->host read for all), the cached
    transposes of those matrices whose entry exists but whose topology has
    changed — what the next backward of each would otherwise rebuild one by
    one, each with its own host read. Called by SET / RigL after a rewrite."""
    stale = []
    for W in Ws:
        cached = _transpose_cache.get(id(W))
        if cached is not None and (cached[0] != W.topology_version or
                                   cached[1] != (int(W.nrows), int(W.ncols))):
            stale.append(W)
    for W, (WT, perm) in zip(stale, transposes_with_perm(stale)):
        _transpose_cache[id(W)] = (W.topology_version, (int(W.nrows), int(W.ncols)), WT, perm)


def _clear_transpose_cache() -> None:
    """Testing utility: clear all cache entries. Not part of the public API."""
    _transpose_cache.clear()


# Phased gather sweep for slk_spmm (slk_csr.phase_lo) where X is far beyond
# the L2s: phases of at most _PHASE_X_ROWS X rows, so that the 1 KB pieces of
# one 256-column tile that a phase gathers (4 MiB) stay in an XCD's L2
# (measured on 16384^2 at 99%: forward 4.10 -> 2.49 ms with 4 phases, 2.90
# with 8, 4.16 with 16). Not for a matrix whose columns are skewed (the
# transpose of one with heavy rows): most of its gathers hit a few hot X rows
# that stay cached anyway, and phases only add passes (the same layer's dX
# 1.75 -> 2.08 ms). slk_spmm uses the bounds only on its 16-byte gather path;
# its LDS-staged kernel, which streams X once per workgroup, ignores them.
_PHASE_MIN_X_BYTES = 128 << 20
_PHASE_X_ROWS = 4096


# Binned slot stream for slk_spmm's LDS-staged kernel (slk_csr.bin_*): for
# matrices without heavy rows where N is large, each staged X element is
# expected to serve at least _BIN_MIN_REUSE rows of a workgroup (density x
# rows per workgroup; fewer, and gathering X rows directly is faster), and a
# wave's rows are expected to hold at most _BIN_MAX_PER_CHUNK slots per
# staged chunk (its window holds 64; a chunk with more takes extra passes).
# Rows per wave and halves are the first of _BIN_SHAPES that qualifies (more
# rows per workgroup stage each X chunk for more rows; two halves halve the
# per-slot overhead per fma). Measured on 16384^2 x 4096 (same bits): the
# 95% layer's input gradient 5.80 -> 5.53 ms at 8 x 2; its forward, whose
# heavy rows run beside the light ones, 6.0 ms on the two-stream path against
# 6.43 binned; at 99% the gather kernel (1.79 ms) beats any binned shape
# (3.5 ms and up: staging all of X per workgroup dominates). Only from
# _BIN_MIN_NNZ live slots: on the 10M- and 60M-GPT layers (0.1-0.5 M slots)
# the binned kernel runs no faster than the LDS kernel, while its build (one
# per topology version; SET rewrites every layer every step) and its view
# cost step time: 60M-GPT + SET 43.0 -> 46.4 ms/step, 10M-GPT 11.1 -> 11.7.
_BIN_MIN_NNZ = 4_000_000
_BIN_MIN_N = 1024
_BIN_MIN_REUSE = 4.0
_BIN_MAX_PER_CHUNK = 48
_BIN_MIN_BLOCKS = 192
_BIN_SHAPES = ((8, 2), (4, 2), (2, 2), (8, 1), (4, 1), (1, 2))


def _bin_shape(W: PaddedCSR, K: int, N: int):
    """(rows per wave, halves) of the binned stream slk_spmm should get for W
    and an N-column X, or None."""
    if N < _BIN_MIN_N or N % 4 or K == 0 or W.nnz < _BIN_MIN_NNZ:
        return None
    first, slots = W._bin_coverage()
    rows = W.nrows - first
    if first > 0 or rows <= 0 or slots <= 0:
        return None
    density = slots / (rows * K)
    for rw, h in _BIN_SHAPES:
        kc = 80 // h
        if -(-K // kc) > _lib.BIN_MAX_CHUNKS:
            continue
        if rw * kc * density > _BIN_MAX_PER_CHUNK or density * 16 * rw < _BIN_MIN_REUSE:
            continue
        if -(-rows // (16 * rw)) * -(-N // (256 * h)) < _BIN_MIN_BLOCKS:
            continue
        return rw, h
    return None


# Schedule overrides for tests and measurement (the launchers' own choices
# otherwise; results keep their bits either way): "spmm_phases" = n forces
# n column phases on slk_spmm's gather path (<= 1: none); "seg" = (block
# columns, slots per segment) forces that segment list on slk_sddmm, () none;
# "bin_shape" = (rows per wave, halves) forces that binned stream on
# slk_spmm, False none.
_overrides: dict[str, object] = {}


def _spmm_view(W: PaddedCSR, X: torch.Tensor):
    """W's view for slk_spmm: with a binned slot stream where it pays (see
    above), else with phase bounds where X is far beyond the L2s and W's
    columns are not skewed."""
    K, N = X.shape
    binned = _overrides.get("bin_shape")
    if binned is None:
        binned = _bin_shape(W, K, N)
    if binned:
        return W._view_binned(*binned)
    forced = _overrides.get("spmm_phases")
    if forced is not None:
        return W._view_phased(int(forced)) if int(forced) > 1 else W._view()
    if 4 * K * N >= _PHASE_MIN_X_BYTES and K > _PHASE_X_ROWS and not W._cols_skewed:
        return W._view_phased(-(-K // _PHASE_X_ROWS))
    return W._view()


def _launch_spmm(W: PaddedCSR, X: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    Y = torch.empty((W.nrows, X.shape[1]), dtype=torch.float32, device=X.device)
    _lib.spmm(_spmm_view(W, X), X, Y, bias)
    return Y


# Segment schedule for dW (slk_csr.seg_start): from this many live slots at
# N >= 1024 (measured per layer: 1.4-1.8x on the 60M-GPT layers, 1.35x on the
# 10M-GPT QKV layer, 1.5x / 1.45x on the 16384^2 layer at 95% / 99%; the
# windowed kernel stays ahead on the 10M-GPT layers of 44-59 k slots).
_SEG_MIN_NNZ = 100_000
# X at least this large (far beyond the 4 MB L2 of an XCD) takes 128-column
# segment blocks where rows are dense enough.
_SEG_WIDE_MIN_X_BYTES = 128 << 20


def _seg_shape(W: PaddedCSR, K: int, N: int) -> tuple[int, int]:
    """(block columns, slots per segment) of the segment list: 128-column
    blocks of 8-slot segments where X is far beyond the L2s (each dY row is
    then fetched once per 128 columns instead of 64; waves skip the slots
    their segments lack, so short runs cost little: 16384^2 at 95% 5.65 ms
    against 6.53 for 64x8, at 99% 1.92 against 2.21 for 64x4); else 64
    columns, with 8 slots per segment where a row holds at least 4 live slots
    per block on average, else 4."""
    if 4 * K * N >= _SEG_WIDE_MIN_X_BYTES:
        return 128, 8
    density = W.nnz / max(1, W.nrows * W.ncols)
    return 64, 8 if density * 64 >= 4 else 4


# Dense rows (slk_csr.n_dense_rows) of a segmented dW run on the matrix cores
# where N is a multiple of 64 (the dense kernel's staged columns) and there
# are at least _DENSE_DW_MIN_ROWS of them: the segment kernel's time follows
# its (row, column block) pairs more than its slots, so a few dense rows
# taken out save little (16384^2 Zipf(1.1) x 4096: 95%, 622 dense rows,
# 5.47 -> 5.22 ms; 99%, 102 rows, 1.86 -> 2.04 ms). "dense_dw" = False in
# _overrides keeps them in the segment list, True takes any count.
_DENSE_DW_N = 64
_DENSE_DW_MIN_ROWS = 256


def _sddmm_view(W: PaddedCSR, X: torch.Tensor):
    """W's view for slk_sddmm: with a segment list where it pays (see above),
    without W's dense rows where the dense kernel takes them."""
    K, N = X.shape
    want = _overrides.get("dense_dw")
    skip = N % _DENSE_DW_N == 0 and N >= _DENSE_DW_N and want is not False and (
        want is True or W._view().n_dense_rows >= _DENSE_DW_MIN_ROWS)
    forced = _overrides.get("seg")
    if forced is not None:
        return W._view_segmented(*forced, skip_dense=skip) if forced else W._view()
    if W.nnz >= _SEG_MIN_NNZ and N >= 1024 and N % 4 == 0:
        return W._view_segmented(*_seg_shape(W, K, N), skip_dense=skip)
    return W._view()


def _launch_sddmm(W: PaddedCSR, dY: torch.Tensor, X: torch.Tensor, kernel: str,
                  dbias: torch.Tensor | None = None) -> torch.Tensor:
    dW = torch.empty(W.total_capacity, dtype=torch.float32, device=X.device)
    order = _lib.SLK_DW_SCALAR if kernel == "scalar" else _lib.SLK_DW_SIMD
    view = _sddmm_view(W, X) if order == _lib.SLK_DW_SIMD else W._view()
    _lib.sddmm(view, dY, X, dW, order, dbias)
    return dW


def _device_f32(t: torch.Tensor) -> torch.Tensor:
    return t.to(dtype=torch.float32).contiguous()


def _check_same_device(W: PaddedCSR, t: torch.Tensor, who: str, name: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{who}: {name} must be on a HIP (ROCm) device (got device={t.device}). "
            f"sparsecore_amd runs the padded-CSR kernels on the GPU only.")
    W._require_device(who)
    if W.device != t.device:
        raise RuntimeError(f"{who}: W is on {W.device} but {name} is on {t.device}")


class _SpMMFunction(torch.autograd.Function):
    """Autograd bridge for Y = W @ X with W a PaddedCSR (ops.py:127-210).

    The first input, ``W_values``, is the tensor autograd tracks (aliased with
    ``W.values`` by SparseLinear); the kernels read the weights through W, as
    the reference does. Backward returns dW aligned with W.values (length
    total_capacity, padding exactly 0) and dX = Wᵀ·dY. A gradient nobody asked
    for (``needs_input_grad`` False) is not computed.
    """

    @staticmethod
    def forward(ctx, W_values, W, X, kernel):
        ctx.save_for_backward(W_values, X)
        ctx.W = W
        ctx.kernel = kernel
        if kernel not in _KERNELS:
            raise ValueError(f"spmm: unknown kernel={kernel!r}. Expected one of: "
                             f"{sorted(_KERNELS)}.")
        _check_same_device(W, X, "spmm", "X")
        return _launch_spmm(W, _device_f32(X))

    @staticmethod
    def backward(ctx, dY):
        W_values, X = ctx.saved_tensors
        dW_values, dX = _spmm_backward(ctx.W, X, _as_row_major(dY), ctx.kernel,
                                       ctx.needs_input_grad[0], ctx.needs_input_grad[2])
        return dW_values, None, dX, None


# Small layers: the backward as one launch (slk_backward_fused) where dW,
# the transpose refresh and dX would each be a few microseconds of launch
# latency (a 512 x 784 layer at N = 256: 6.8 + 2.3 + 8.2 us in a graph): up
# to this many waves in the fused grid, one round of waves on the chip.
_FUSED_MAX_WAVES = 8192


def _fused_backward(W: PaddedCSR, N: int, kernel: str) -> bool:
    forced = _overrides.get("fused_backward")
    if forced is not None:
        return bool(forced) and kernel != "scalar"
    if kernel == "scalar" or N == 0:
        return False
    waves = W.ncols * -(-N // 64) + -(-W.total_capacity // 16)
    return waves <= _FUSED_MAX_WAVES


def _spmm_backward(W: PaddedCSR, X: torch.Tensor, dY_f32: torch.Tensor, kernel: str,
                   need_dw: bool, need_dx: bool, dbias: torch.Tensor | None = None):
    """dW on the live slots (SDDMM) and dX = Wᵀ·dY through the transpose cache
    (ops.py:167-210); a gradient that is not needed is not computed. With
    ``dbias`` (and dW needed) the dW launch also writes dY's row sums there.
    Small layers run both in one launch, W's values read through the
    transpose's slot map instead of a refresh (same bits)."""
    if need_dw and need_dx and _fused_backward(W, dY_f32.shape[1], kernel):
        WT, perm = _cached_transpose_structure(W)
        X32 = _device_f32(X)
        dW_values = torch.empty(W.total_capacity, dtype=torch.float32, device=X32.device)
        dX = torch.empty(W.ncols, dY_f32.shape[1], dtype=torch.float32, device=X32.device)
        _lib.backward_fused(W._view(), WT._view(), perm, dY_f32, X32, dW_values, dbias, dX)
        return dW_values, dX
    dW_values = dX = None
    if need_dw:
        dW_values = _launch_sddmm(W, dY_f32, _device_f32(X), kernel, dbias)
    if need_dx:
        WT = _cached_transpose(W)
        dX = _launch_spmm(WT, dY_f32)
    return dW_values, dX


def _as_row_major(t: torch.Tensor) -> torch.Tensor:
    """``t.to(float32).contiguous()`` where a transposed view is copied by the
    library's tiled transpose (slk_transpose_dense) instead of torch's
    strided copy: the `dY.contiguous()` of ops.py:174, bit for bit."""
    t = t.to(dtype=torch.float32)
    if t.is_contiguous():
        return t
    if t.dim() == 2 and t.t().is_contiguous() and t.device.type == "cuda":
        out = torch.empty(t.shape, dtype=torch.float32, device=t.device)
        _lib.transpose_dense(t.t(), out)
        return out
    return t.contiguous()


def _narrow_layer(W: PaddedCSR) -> bool:
    """A layer small enough for the narrow path (slk_spmm_t forward,
    slk_backward_narrow backward): at most 64 output rows and 8192 slots."""
    return W.nrows <= _lib.NARROW_MAX_ROWS and W.total_capacity <= _lib.NARROW_MAX_CAPACITY


class _SparseLinearFunction(torch.autograd.Function):
    """SparseLinear's ``Y = W @ x_flatᵀ (+ bias[:, None])`` as one autograd node
    (sparselab/nn.py:229-241 with ops.py:127-210 inside).

    Takes the token-major input x_flat (N x K). Returns Y feature-major
    (M x N), whose ``.t()`` is the layer output, or — for a narrow layer
    (``_narrow_layer``) — the layer output itself, token-major (N x M)
    contiguous. The layout changes of the reference (``x_flat.t().contiguous()``,
    the bias add, ``dY.contiguous()``) are done by the library: the transpose
    by slk_transpose_dense — free when x_flat is the transposed view a
    previous SparseLinear returned — and the bias add inside the SpMM store
    (slk_spmm_bias / slk_spmm_t: the bits of the separate float32 add).
    Backward is ``_SpMMFunction``'s, plus dbias = Σ_n dY[:, n] computed in the
    dW launch (slk_sddmm_bias); a narrow layer does all three gradients in one
    launch from the token-major gradient (slk_backward_narrow), with no
    transpose cache. dx is returned as the transposed view of dX (K x N).
    """

    @staticmethod
    def forward(ctx, W_values, bias, W, x_flat, kernel):
        if kernel not in _KERNELS:
            raise ValueError(f"spmm: unknown kernel={kernel!r}. Expected one of: "
                             f"{sorted(_KERNELS)}.")
        _check_same_device(W, x_flat, "spmm", "X")
        X = _as_row_major(x_flat.t())
        if bias is not None:
            _check_same_device(W, bias, "spmm", "bias")
            if bias.dtype != torch.float32 or bias.shape != (W.nrows,):
                raise ValueError(f"spmm: bias must be float32 of shape ({W.nrows},), got "
                                 f"{bias.dtype} {tuple(bias.shape)}")
            bias = bias.contiguous()
        ctx.save_for_backward(W_values, X)
        ctx.W = W
        ctx.kernel = kernel
        ctx.narrow = _narrow_layer(W)
        if ctx.narrow:
            Yt = torch.empty(X.shape[1], W.nrows, dtype=torch.float32, device=X.device)
            _lib.spmm_t(W._view(), X, Yt, bias)
            return Yt
        return _launch_spmm(W, X, bias)

    @staticmethod
    def backward(ctx, dY):
        W_values, X = ctx.saved_tensors
        if ctx.narrow:
            return _narrow_backward(ctx, X, dY)
        dY_f32 = _as_row_major(dY)
        need_dw, need_db = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dbias = None
        if need_db:  # fused into the dW launch when dW is computed too
            dbias = torch.empty(dY_f32.shape[0], dtype=torch.float32, device=dY_f32.device)
            if not need_dw:
                torch.sum(dY_f32, dim=1, out=dbias)
        dW_values, dX = _spmm_backward(ctx.W, X, dY_f32, ctx.kernel, need_dw,
                                       ctx.needs_input_grad[3], dbias if need_dw else None)
        return dW_values, dbias, None, (dX.t() if dX is not None else None), None


def _narrow_backward(ctx, X: torch.Tensor, dYt: torch.Tensor):
    """Gradients of a narrow layer from the token-major output gradient."""
    W = ctx.W
    dev = X.device
    dYt = dYt.to(torch.float32).contiguous()
    need_dw, need_db, need_dx = (ctx.needs_input_grad[0], ctx.needs_input_grad[1],
                                 ctx.needs_input_grad[3])
    dW = torch.empty(W.total_capacity, dtype=torch.float32, device=dev) if need_dw else None
    dbias = torch.empty(W.nrows, dtype=torch.float32, device=dev) if need_db else None
    dX = torch.empty(X.shape, dtype=torch.float32, device=dev) if need_dx else None
    order = _lib.SLK_DW_SCALAR if ctx.kernel == "scalar" else _lib.SLK_DW_SIMD
    _lib.backward_narrow(W._view(), dYt, X, dW, dbias, dX, order)
    return dW, dbias, None, (dX.t() if dX is not None else None), None


def spmm(W: PaddedCSR, X: torch.Tensor, *, kernel: str = "auto") -> torch.Tensor:
    """Y = W @ X for a PaddedCSR W (M x K) and a dense 2-D X (K x N) on the GPU.

    Same contract as sparselab.ops.spmm (ops.py:217-331) except for the
    device: X (and W) must live on the HIP device. Any float dtype is
    converted to float32. If X requires grad the call goes through the
    autograd Function. ``kernel`` ("auto", "simd", "scalar") selects the dW
    summation order of the reference kernel of that name; the forward result
    is the same for all three.

    Raises TypeError (wrong W / X type), RuntimeError (tensor not on the HIP
    device) and ValueError (X not 2-D, shape mismatch, unknown kernel).
    """
    if not isinstance(W, PaddedCSR):
        raise TypeError(f"spmm: W must be a sparselab.PaddedCSR, got {type(W).__name__}")
    if not isinstance(X, torch.Tensor):
        raise TypeError(f"spmm: X must be a torch.Tensor, got {type(X).__name__}")
    if X.device.type != "cuda":
        raise RuntimeError(
            f"spmm: X must be on a HIP (ROCm) device (got device={X.device}). "
            f"sparsecore_amd runs the padded-CSR kernels on the GPU only.")
    if X.dim() != 2:
        raise ValueError(f"spmm: X must be 2-D, got shape={tuple(X.shape)}")
    if kernel not in _KERNELS:
        raise ValueError(f"spmm: unknown kernel={kernel!r}. Expected one of: "
                         f"{sorted(_KERNELS)}.")
    _check_same_device(W, X, "spmm", "X")
    X_f32 = _device_f32(X)
    W_values_t = W.values
    if X_f32.requires_grad or W_values_t.requires_grad:
        return _SpMMFunction.apply(W_values_t, W, X_f32, kernel)
    return _launch_spmm(W, X_f32)


def dense_grad(dY: torch.Tensor, X: torch.Tensor) -> torch.Tensor:
    """G = dY @ Xᵀ (M x K) for dense dY (M x N) and X (K x N) on the GPU.

    Mirrors ``_core.dense_grad`` (csrc/bindings.cpp:445-485): 2-D inputs,
    converted to contiguous float32, ValueError on a rank or inner-dimension
    mismatch with the reference's message. Every element is the reference
    build's running sum over N in order, so G is bit-identical to
    csrc/kernels/dense_grad.cpp:57-83.
    """
    for name, t in (("dY", dY), ("X", X)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"dense_grad: {name} must be a torch.Tensor, got {type(t).__name__}")
        if t.dim() != 2:
            raise ValueError(f"dense_grad: {name} must be 2-D, got ndim={t.dim()}.")
        if t.device.type != "cuda":
            raise RuntimeError(f"dense_grad: {name} must be on a HIP (ROCm) device "
                               f"(got device={t.device}).")
    if dY.device != X.device:
        raise RuntimeError(f"dense_grad: dY is on {dY.device} but X is on {X.device}")
    M, N = dY.shape
    K, N_x = X.shape
    if N != N_x:
        raise ValueError(f"dense_grad: dY.shape[1]={N} must equal X.shape[1]={N_x} "
                         f"(shared inner dim N).")
    G = torch.empty((M, K), dtype=torch.float32, device=dY.device)
    _lib.dense_grad(_device_f32(dY), _device_f32(X), M, K, N, False, G)
    return G


def _dense_grad_token_major(dy: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """G = dyᵀ @ x for token-major dy (N x M) and x (N x K): the same G as
    ``dense_grad(dy.t(), x.t())``, bit for bit, without the transpose copies."""
    N, M = dy.shape
    K = x.shape[1]
    G = torch.empty((M, K), dtype=torch.float32, device=dy.device)
    _lib.dense_grad(_device_f32(dy), _device_f32(x), M, K, N, True, G)
    return G
