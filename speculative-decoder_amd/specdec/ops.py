"""Tensor-level wrappers of the libspecdec.so entry points.

Each wrapper checks devices, dtypes and contiguity on the host, launches on
torch's current HIP stream and raises on a non-zero status.  Nothing here
computes on the CPU: inputs that are not on a GPU are an error.
"""
from __future__ import annotations

import torch

from specdec._lib import lib

OK, EINVAL, EHIP, EUNSUPPORTED, ENOSCRATCH = 0, 1, 2, 3, 4
F32, F64, BF16 = 0, 1, 2

_DTYPES = {torch.float32: F32, torch.float64: F64, torch.bfloat16: BF16}


class KernelError(RuntimeError):
    pass


def _check(status: int, name: str) -> None:
    if status == OK:
        return
    what = {EINVAL: "invalid argument", EHIP: "HIP launch failed", EUNSUPPORTED: "unsupported shape",
            ENOSCRATCH: "needs more split partials than the library's static buffer holds"}
    err = NotImplementedError if status == EUNSUPPORTED else KernelError
    raise err(f"{name}: {what.get(status, 'error')} (status {status})")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def gpu(t: torch.Tensor, name: str = "tensor") -> torch.Tensor:
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be on a GPU (got {t.device}); the hot path has no CPU fallback")
    return t


def _on(dev: torch.device, t: torch.Tensor, name: str, dtype: torch.dtype | None = None,
        contiguous: bool = False, numel: int | None = None) -> torch.Tensor:
    """Host-side check of a tensor whose pointer goes to a kernel: on `dev`,
    of `dtype`, contiguous, holding `numel` elements, as asked.  A pointer to
    host memory or a short buffer would otherwise become a GPU memory fault."""
    if t.device != dev:
        raise RuntimeError(f"{name} must be on {dev} (got {t.device}); the hot path has no CPU fallback")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{name} must hold {numel} elements (got {t.numel()})")
    return t


def _token_rows(t: torch.Tensor, tokens: int, stride: int, row: int, name: str) -> None:
    """Host-side check that t's memory, from its first element, holds `tokens`
    rows of `row` elements `stride` apart (the rows a kernel reads or writes
    through t's pointer and the stride it is given)."""
    if tokens <= 0:
        return
    if stride < row:
        raise ValueError(f"{name}: a token stride of {stride} is shorter than a token's {row} elements")
    have = t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()
    need = (tokens - 1) * stride + row
    if need > have:
        raise ValueError(f"{name} holds {have} elements from its start; {tokens} token rows of {row} "
                         f"elements at stride {stride} need {need}")


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------ accept --
def probabilities(logits: torch.Tensor, temperature: float, out: torch.Tensor | None = None,
                  index_out: torch.Tensor | None = None) -> torch.Tensor:
    """[..., V] logits -> fp32 probabilities (one-hot argmax at temperature
    0).  `out` may be a row-strided view to write into (rows of V fp32 with
    unit inner stride); at temperature 0 `index_out` (int64, one per row,
    any row stride) receives each row's argmax."""
    gpu(logits, "logits")
    shape = logits.shape
    x = logits.reshape(-1, shape[-1])
    if x.stride(-1) != 1:
        x = x.contiguous()
    rows, v = x.shape
    fresh = out is None
    if fresh:
        out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    _on(x.device, out, "out")
    o2 = out if out.dim() == 2 else out.view(rows, v)
    if o2.dtype != torch.float32 or tuple(o2.shape) != (rows, v) or o2.stride(-1) != 1:
        raise ValueError("out must be fp32 [rows, V] with unit inner stride")
    idx_ptr, idx_stride = None, 0
    if index_out is not None:
        if temperature != 0.0:
            raise ValueError("index_out is defined at temperature 0 only")
        _on(x.device, index_out, "index_out", torch.int64, numel=rows)
        if index_out.dim() > 1 and not index_out.is_contiguous():
            raise ValueError("index_out must be a vector or contiguous")
        idx_ptr, idx_stride = index_out.data_ptr(), (index_out.stride(0) if index_out.dim() else 1)
    st = lib().specdec_probabilities(x.data_ptr(), dtype_code(x), rows, v, x.stride(0), float(temperature),
                                     o2.data_ptr(), o2.stride(0), idx_ptr, idx_stride, stream())
    _check(st, "probabilities")
    return out.view(shape) if fresh else out


def _rows3(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) != 1:
        t = t.contiguous()
    return t


def _accept_inputs(p, q, draft, u_accept) -> tuple[int, int]:
    """Shapes and devices of the accept inputs: p [B, k+1, V], q [B, k, V] of
    p's dtype, draft int64 [B, k] and u_accept [B, k] (p's dtype), contiguous."""
    b, k = draft.shape
    if p.dim() != 3 or q.dim() != 3 or tuple(p.shape[:2]) != (b, k + 1) or tuple(q.shape) != (b, k, p.shape[2]):
        raise ValueError(f"p must be [B, k+1, V] and q [B, k, V] for draft [B, k] = [{b}, {k}] "
                         f"(got p {tuple(p.shape)}, q {tuple(q.shape)})")
    _on(p.device, q, "q", p.dtype)
    _on(p.device, draft, "draft", torch.int64, True)
    _on(p.device, u_accept, "u_accept", p.dtype, True, b * k)
    return b, k


class AcceptWorkspace:
    """Grow-only workspace of the many-CU accept-reject (arrival counters,
    the call epoch and the meeting words), zeroed when it is allocated and
    never cleared again: every word a call reads carries that call's tag.
    Calls sharing one must be ordered on one stream."""

    def __init__(self, device: torch.device) -> None:
        self.device = device
        self.buf = torch.zeros(0, dtype=torch.uint8, device=device)

    def reserve(self, batch: int) -> torch.Tensor:
        import ctypes

        nbytes = ctypes.c_int64()
        _check(lib().specdec_accept_workspace(batch, ctypes.byref(nbytes)), "accept_workspace")
        if nbytes.value > self.buf.numel():
            self.buf = torch.zeros(max(nbytes.value, 2 * self.buf.numel()), dtype=torch.uint8, device=self.device)
        return self.buf


_accept_workspaces: dict[torch.device, AcceptWorkspace] = {}


def accept_workspace_for(device: torch.device) -> AcceptWorkspace:
    ws = _accept_workspaces.get(device)
    if ws is None:
        ws = _accept_workspaces[device] = AcceptWorkspace(device)
    return ws


# Reads of the values a many-CU accept workgroup waits for, after its first,
# before it computes the missing chunks itself (about a microsecond each).
ACCEPT_SPIN = 1 << 14


def accept_reject(p, q, draft, u_accept, u_residual, workspace: AcceptWorkspace | None = None,
                  single: bool = False, spin: int = ACCEPT_SPIN) -> torch.Tensor:
    """Fused accept + residual + inverse CDF; returns int64 [3, B] on the GPU:
    n_accepted, next_token, and a flag that is 1 for a drafted token with
    zero q(x) or outside the vocabulary.  `single` asks for the
    one-workgroup-per-row kernel (no workspace); `spin` bounds the waits of
    the many-CU kernel (negative: none; every workgroup then computes the
    other chunks' values itself, with the same bits)."""
    p, q = _rows3(gpu(p, "p")), _rows3(gpu(q, "q"))
    b, k = _accept_inputs(p, q, draft, u_accept)
    _on(p.device, u_residual, "u_residual", p.dtype, True, b)
    out = torch.empty(3, b, dtype=torch.int64, device=p.device)
    ws_ptr, ws_bytes = None, 0
    if not single:
        buf = (workspace or accept_workspace_for(p.device)).reserve(b)
        ws_ptr, ws_bytes = buf.data_ptr(), buf.numel()
    st = lib().specdec_accept_reject(p.data_ptr(), q.data_ptr(), dtype_code(p), p.stride(0), p.stride(1),
                                     q.stride(0), q.stride(1), draft.data_ptr(), u_accept.data_ptr(),
                                     u_residual.data_ptr(), b, k, p.shape[-1], out.data_ptr(), ws_ptr, ws_bytes,
                                     int(spin), stream())
    _check(st, "accept_reject")
    return out


def accept_reject_logits(target_logits, draft_logits, temperature: float, draft, u_accept, u_residual,
                         workspace: AcceptWorkspace | None = None, spin: int = ACCEPT_SPIN) -> torch.Tensor | None:
    """probabilities() of the target [B, k+1, V] and draft [B, k, V] fp32
    logits followed by accept_reject, in one launch that reads the logits
    once; int64 [3, B] as accept_reject returns, or None when the shapes do
    not fit the kernel (more than 16 drafted positions, rows that are not
    16-byte aligned, too many rows for the GPU)."""
    tl, dl = _rows3(gpu(target_logits, "target_logits")), _rows3(gpu(draft_logits, "draft_logits"))
    if tl.dtype != torch.float32:
        return None
    b, k = _accept_inputs(tl, dl, draft, u_accept)
    _on(tl.device, u_residual, "u_residual", tl.dtype, True, b)
    if temperature < 0:
        raise ValueError(f"temperature must be >= 0 (got {temperature})")
    out = torch.empty(3, b, dtype=torch.int64, device=tl.device)
    buf = (workspace or accept_workspace_for(tl.device)).reserve(b)
    st = lib().specdec_accept_reject_logits(tl.data_ptr(), dl.data_ptr(), dtype_code(tl), tl.stride(0), tl.stride(1),
                                            dl.stride(0), dl.stride(1), float(temperature), draft.data_ptr(),
                                            u_accept.data_ptr(), u_residual.data_ptr(), b, k, tl.shape[-1],
                                            out.data_ptr(), buf.data_ptr(), buf.numel(), int(spin), stream())
    if st == EUNSUPPORTED:
        return None
    _check(st, "accept_reject_logits")
    return out


def accept_count(p, q, draft, u_accept) -> torch.Tensor:
    """Accept stage alone; int64 [2, B]: n_accepted, and a flag for a zero
    q(x) or a draft id outside the vocabulary."""
    p, q = _rows3(gpu(p, "p")), _rows3(gpu(q, "q"))
    b, k = _accept_inputs(p, q, draft, u_accept)
    out = torch.empty(2, b, dtype=torch.int64, device=p.device)
    st = lib().specdec_accept_count(p.data_ptr(), q.data_ptr(), dtype_code(p), p.stride(0), p.stride(1),
                                    q.stride(0), q.stride(1), draft.data_ptr(), u_accept.data_ptr(), b, k,
                                    p.shape[-1], out.data_ptr(), stream())
    _check(st, "accept_count")
    return out


def sample_inverse_cdf(probs: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    gpu(probs, "probs")
    if probs.stride(-1) != 1:
        probs = probs.contiguous()
    b, v = probs.shape
    _on(probs.device, u, "u", probs.dtype, True, b)
    out = torch.empty(b, dtype=torch.int64, device=probs.device)
    st = lib().specdec_sample_inverse_cdf(probs.data_ptr(), dtype_code(probs), b, v, probs.stride(0),
                                          u.data_ptr(), out.data_ptr(), stream())
    _check(st, "sample_inverse_cdf")
    return out


def one_hot(ids: torch.Tensor, vocab: int) -> torch.Tensor:
    gpu(ids, "ids")
    flat = ids.reshape(-1).to(torch.int64).contiguous()
    out = torch.empty(flat.numel(), vocab, dtype=torch.float32, device=ids.device)
    _check(lib().specdec_one_hot(flat.data_ptr(), flat.numel(), vocab, out.data_ptr(), stream()), "one_hot")
    return out.view(*ids.shape, vocab)


# -------------------------------------------------------------------- head --
# rows of one fused head call (hidden rows whose probabilities one launch
# writes), at most
HEAD_FUSED_ROWS = 16
# polls of the fused head's meeting before a workgroup computes the missing
# statistics itself (about 0.2 us each)
HEAD_SPIN = 1 << 17
_head_workspaces: dict[torch.device, torch.Tensor] = {}


def head_workspace(device: torch.device) -> torch.Tensor:
    """The fused head's meeting slots on `device`: allocated zeroed once, never
    cleared or reallocated (graph captures keep its address).  Calls sharing
    it must be ordered on one stream."""
    ws = _head_workspaces.get(device)
    if ws is None:
        import ctypes

        nbytes = ctypes.c_int64()
        _check(lib().specdec_head_workspace(ctypes.byref(nbytes)), "head_workspace")
        ws = _head_workspaces[device] = torch.zeros(nbytes.value, dtype=torch.uint8, device=device)
    return ws


def _head_operands(x: torch.Tensor, w: torch.Tensor) -> tuple[torch.Tensor, int]:
    gpu(w, "w")
    _on(w.device, x, "hidden", torch.bfloat16)
    if w.dtype != torch.bfloat16 or w.dim() != 2 or not w.is_contiguous():
        raise ValueError("the head must be a contiguous bf16 [V, H] tensor")
    h = w.shape[1]
    if x.shape[-1] != h:
        raise ValueError(f"hidden rows have {x.shape[-1]} features, the head {h}")
    x2 = x.reshape(-1, h)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2, x2.shape[0]


def _rows_out(out: torch.Tensor | None, rows: int, v: int, dev: torch.device, name: str) -> torch.Tensor:
    """`out` as an fp32 [rows, V] view with unit inner stride (any row stride)."""
    if out is None:
        return torch.empty(rows, v, dtype=torch.float32, device=dev)
    _on(dev, out, name, torch.float32)
    o2 = out if out.dim() == 2 else out.view(rows, v)
    if tuple(o2.shape) != (rows, v) or o2.stride(-1) != 1:
        raise ValueError(f"{name} must be fp32 [rows, V] with unit inner stride")
    return o2


LINEAR_ROWS = 64  # rows of a specdec_linear call, at most
W_ROWS, W_TILED = 0, 1  # weight layouts of the linear entries


def tile_weight(w: torch.Tensor) -> torch.Tensor:
    """W [N, K] (N % 16 == 0, K % 32 == 0) in the tiled layout, as
    [N/16, K/32, 4, 16, 8]: the 16 x 32 block of feature tile t and k-step
    s is 1 KB contiguous, lane (c, g) of a wave holding row 16t + c at
    k = 32s + 8g .. 32s + 8g + 7, so each load instruction of the linear
    kernels reads one contiguous KB.  The projection's bits are the same as
    with W itself.  Made once per weight; prompt-sized GEMMs keep W."""
    n, k = w.shape
    if n % 16 or k % 32:
        raise ValueError(f"a tiled weight needs N % 16 == 0 and K % 32 == 0 (got {n} x {k})")
    return w.reshape(n // 16, 16, k // 32, 4, 8).permute(0, 2, 3, 1, 4).contiguous()


def _weight(w: torch.Tensor) -> tuple[int, int, int]:
    """(N, K, layout) of a linear weight: W [N, K] row-major (contiguous) or
    its `tile_weight` form."""
    if w.dim() == 5 and tuple(w.shape[2:]) == (4, 16, 8) and w.is_contiguous():
        return w.shape[0] * 16, w.shape[1] * 32, W_TILED
    if w.dim() == 2 and w.is_contiguous():
        return w.shape[0], w.shape[1], W_ROWS
    raise ValueError("w must be a contiguous [N, K] tensor or a tile_weight() result")


def linear_fits(x: torch.Tensor, w: torch.Tensor) -> bool:
    """Whether `linear` takes x @ w.T: bf16, at most LINEAR_ROWS rows, the
    inner size a multiple of 32 up to 8192, a contiguous (or tiled) weight."""
    if w.dtype != torch.bfloat16 or not (w.dim() == 2 and w.is_contiguous() or w.dim() == 5):
        return False
    k = _weight(w)[1]
    return x.dtype == torch.bfloat16 and k % 32 == 0 and k <= 8192 and x.numel() // k <= LINEAR_ROWS and x.is_cuda


def linear(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None, accumulate: bool = False) -> torch.Tensor:
    """x [..., K] bf16 times w [N, K] bf16 (or its `tile_weight` form)
    transposed, accumulated in fp32 and rounded once: bf16 [..., N].  With
    `accumulate`, out += x @ w.T inside that rounding.  A row's result does
    not depend on the other rows of the call."""
    gpu(w, "w")
    _on(w.device, x, "x", torch.bfloat16)
    if w.dtype != torch.bfloat16:
        raise ValueError("w must be bf16")
    n, k, layout = _weight(w)
    if x.shape[-1] != k:
        raise ValueError(f"x rows have {x.shape[-1]} features, w {k}")
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    rows = x2.shape[0]
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs an out to add to")
        o2 = torch.empty(rows, n, dtype=torch.bfloat16, device=w.device)
    else:
        _on(w.device, out, "out", torch.bfloat16)
        o2 = out.view(rows, n) if out.dim() != 2 else out
        if tuple(o2.shape) != (rows, n) or o2.stride(-1) != 1:
            raise ValueError("out must be bf16 [rows, N] with unit inner stride")
    st = lib().specdec_linear(x2.data_ptr(), x2.stride(0), w.data_ptr(), k, layout, rows, k, n, o2.data_ptr(),
                              o2.stride(0),
                              int(accumulate), stream())
    _check(st, "linear")
    return o2.view(*x.shape[:-1], n) if out is None else out


def linear_silu(x: torch.Tensor, w: torch.Tensor, hidden: torch.Tensor, out: torch.Tensor, eps: float) -> torch.Tensor:
    """rms_silu_mul(linear(x, w), hidden, out, eps) in one launch, with the
    same bits: w is the fused [2 I, K] gate/up weight (or its `tile_weight`
    form), out bf16 [..., I]."""
    gpu(w, "w")
    _on(w.device, x, "x", torch.bfloat16)
    _on(w.device, hidden, "hidden", torch.bfloat16)
    _on(w.device, out, "out", torch.bfloat16)
    n2, k, layout = _weight(w)
    if w.dtype != torch.bfloat16 or n2 % 2:
        raise ValueError("w must be a bf16 [2 I, K] tensor")
    inter = n2 // 2
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    rows = x2.shape[0]
    h2 = hidden.reshape(rows, -1)
    if h2.stride(-1) != 1 or h2.stride(0) % 8 or h2.data_ptr() % 16:
        h2 = h2.contiguous()
    o2 = out.view(rows, inter) if out.dim() != 2 else out
    if tuple(o2.shape) != (rows, inter) or o2.stride(-1) != 1:
        raise ValueError("out must be bf16 [rows, I] with unit inner stride")
    st = lib().specdec_linear_silu(x2.data_ptr(), x2.stride(0), w.data_ptr(), k, layout, rows, k, inter, h2.data_ptr(),
                                   h2.stride(0), h2.shape[1], float(eps), o2.data_ptr(), o2.stride(0), stream())
    _check(st, "linear_silu")
    return out


def head_logits(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., H] bf16 times the head w [V, H] bf16, accumulated in fp32:
    fp32 logits [..., V].  A row's logits do not depend on the other rows
    of the call."""
    x2, rows = _head_operands(x, w)
    v = w.shape[0]
    o2 = _rows_out(out, rows, v, w.device, "out")
    st = lib().specdec_head_logits(x2.data_ptr(), x2.stride(0), w.data_ptr(), w.shape[1], rows, w.shape[1], v,
                                   o2.data_ptr(), o2.stride(0), stream())
    _check(st, "head_logits")
    return o2.view(*x.shape[:-1], v) if out is None else out


def head_probabilities(x: torch.Tensor, w: torch.Tensor, temperature: float, out: torch.Tensor | None = None,
                       index_out: torch.Tensor | None = None, logits_out: torch.Tensor | None = None,
                       spin: int = HEAD_SPIN) -> torch.Tensor:
    """probabilities(head_logits(x, w), temperature) in one launch, at most
    HEAD_FUSED_ROWS hidden rows: fp32 [..., V], the one-hot of each row's
    argmax (lowest id among ties) at temperature 0, else softmax(logits / T).
    `index_out` (int64, one per row) receives the argmax at temperature 0;
    `logits_out` the logits, the bits head_logits gives."""
    x2, rows = _head_operands(x, w)
    if rows > HEAD_FUSED_ROWS:
        raise ValueError(f"a fused head call takes at most {HEAD_FUSED_ROWS} rows (got {rows})")
    v = w.shape[0]
    fresh = out is None
    o2 = _rows_out(out, rows, v, w.device, "out")
    l2 = None if logits_out is None else _rows_out(logits_out, rows, v, w.device, "logits_out")
    idx_ptr, idx_stride = None, 0
    if index_out is not None:
        if temperature != 0.0:
            raise ValueError("index_out is defined at temperature 0 only")
        _on(w.device, index_out, "index_out", torch.int64, numel=rows)
        if index_out.dim() > 1 and not index_out.is_contiguous():
            raise ValueError("index_out must be a vector or contiguous")
        idx_ptr, idx_stride = index_out.data_ptr(), (index_out.stride(0) if index_out.dim() else 1)
    ws = head_workspace(w.device)
    st = lib().specdec_head_probabilities(x2.data_ptr(), x2.stride(0), w.data_ptr(), w.shape[1], rows, w.shape[1], v,
                                          float(temperature), o2.data_ptr(), o2.stride(0), idx_ptr, idx_stride,
                                          ptr(l2), 0 if l2 is None else l2.stride(0), ws.data_ptr(), ws.numel(),
                                          int(spin), stream())
    _check(st, "head_probabilities")
    return o2.view(*x.shape[:-1], v) if fresh else out


def head_fused(w: torch.Tensor, rows: int, fastest: bool = False) -> bool:
    """Whether head_probabilities takes `rows` hidden rows against head w on
    this GPU (bf16, H a multiple of 32 up to 2048, the vocab spread over at
    most one workgroup per compute unit with at most 16 tiles of 16 each).
    With `fastest`, also whether the one fused launch is at least as fast as
    head_logits followed by the softmax kernel on MI355X (kernel traces of
    graph replays, W from HBM): up to 5 rows of a 2048-wide head (52.9 against
    53.1 us at 5 rows, 51.9 against 51.9 at 1) and a single row of a narrower
    one (576 wide: 22.3 against 22.2 us at 1 row, 22.8 against 22.0 at 5).
    Its exchange of per-slice statistics grows with the rows; the pair does
    not."""
    if w.dtype != torch.bfloat16 or w.dim() != 2 or not (1 <= rows <= HEAD_FUSED_ROWS):
        return False
    if fastest and rows > (5 if w.shape[1] >= 1024 else 1):
        return False
    v, h = w.shape
    if h % 32 or h > 2048 or v * h * 2 > 2**31 - 1:
        return False
    cus = torch.cuda.get_device_properties(w.device).multi_processor_count
    tiles = -(-v // 16)
    tpw = max(1, -(-tiles // cus))
    return tpw <= 16 and -(-tiles // tpw) <= min(cus, 256)


# ------------------------------------------------------------------ n-gram --
def ngram_lookup(history: torch.Tensor, lengths: torch.Tensor, k: int, max_n: int):
    """history int32 [B, cap], lengths int32 [B] -> (draft int64 [B, k], match int32 [B, 2])."""
    gpu(history, "history")
    if history.dtype != torch.int32 or history.dim() != 2 or history.stride(1) != 1:
        raise ValueError("history must be int32 [B, capacity] with unit inner stride")
    b = history.shape[0]
    _on(history.device, lengths, "lengths", torch.int32, True, b)
    draft = torch.empty(b, k, dtype=torch.int64, device=history.device)
    match = torch.empty(b, 2, dtype=torch.int32, device=history.device)
    st = lib().specdec_ngram_lookup(history.data_ptr(), history.stride(0), lengths.data_ptr(), b, k, max_n,
                                    draft.data_ptr(), match.data_ptr(), stream())
    _check(st, "ngram_lookup")
    return draft, match


# ------------------------------------------------------------------- cache --
def _tables(tables: torch.Tensor) -> torch.Tensor:
    gpu(tables, "tables")
    if tables.dtype != torch.int32 or tables.dim() != 2 or tables.stride(1) != 1:
        raise ValueError("block tables must be int32 [rows, capacity] with unit inner stride")
    return tables


def _meta(dev: torch.device, meta: torch.Tensor, batch: int) -> torch.Tensor:
    """Per-call row metadata: int32 [3, batch] (table row, cached length, new tokens)."""
    return _on(dev, meta, "meta", torch.int32, True, 3 * batch)


def _stack_and_marks(free_stack: torch.Tensor, used: torch.Tensor) -> None:
    _on(free_stack.device, free_stack, "free_stack", torch.int32, True)
    _on(free_stack.device, used, "used", torch.uint8, True)
    if used.numel() < free_stack.numel():
        raise ValueError("used needs a mark per block")


def block_plan(tables, free_stack, used, top: int, entries, n_push: int, n_pop: int, popped=None) -> None:
    dev = gpu(tables, "tables").device
    _tables(tables)
    _stack_and_marks(free_stack, used)
    _on(dev, entries, "entries", torch.int32, True)
    if popped is not None:
        _on(dev, popped, "popped", torch.int32, True)
    st = lib().specdec_block_plan(tables.data_ptr(), tables.stride(0), free_stack.data_ptr(), used.data_ptr(),
                                  free_stack.numel(), top, entries.data_ptr(), n_push, n_pop, ptr(popped),
                                  stream())
    _check(st, "block_plan")


def block_free_checked(free_stack, used, top: int, block: int, status) -> None:
    dev = gpu(free_stack, "free_stack").device
    _stack_and_marks(free_stack, used)
    _on(dev, status, "status", torch.int32)
    st = lib().specdec_block_free_checked(free_stack.data_ptr(), used.data_ptr(), free_stack.numel(), top,
                                          block, status.data_ptr(), stream())
    _check(st, "block_free_checked")


def block_slots(row: torch.Tensor, start: int, stop: int, block_size: int) -> torch.Tensor:
    gpu(row, "row")
    if row.dtype != torch.int32 or (stop > start and row.numel() * block_size < stop):
        raise ValueError("row must be int32 holding a block for every position below stop")
    out = torch.empty(max(stop - start, 0), dtype=torch.int64, device=row.device)
    st = lib().specdec_block_slots(row.data_ptr(), start, stop, block_size, out.data_ptr(), stream())
    _check(st, "block_slots")
    return out


def slot_map(tables, meta, batch: int, block_size: int, width: int, read_width: int, write_offsets,
             n_write: int):
    dev = _tables(tables).device
    _meta(dev, meta, batch)
    _on(dev, write_offsets, "write_offsets", torch.int32, True, batch)
    write = torch.empty(n_write, dtype=torch.int64, device=dev)
    write_index = torch.empty(n_write, dtype=torch.int64, device=dev)
    read = torch.empty(batch, read_width, dtype=torch.int64, device=dev)
    st = lib().specdec_slot_map(tables.data_ptr(), tables.stride(0), meta.data_ptr(), batch, block_size, width,
                                read_width, write_offsets.data_ptr(), write.data_ptr(), write_index.data_ptr(),
                                read.data_ptr(), stream())
    _check(st, "slot_map")
    return write, write_index, read


def rope_append(qkv, n_heads, n_kv_heads, head_dim, cos, sin, meta, batch, width, tables, block_size,
                k_pool, v_pool) -> None:
    dev = gpu(qkv, "qkv").device
    _qkv_side(dev, qkv, cos, sin, meta, batch, width, tables, k_pool, v_pool)
    _token_rows(qkv, batch * width, qkv.stride(1), (n_heads + 2 * n_kv_heads) * head_dim, "qkv")
    st = lib().specdec_rope_append(qkv.data_ptr(), dtype_code(qkv), qkv.stride(1), n_heads, n_kv_heads, head_dim,
                                   cos.data_ptr(), sin.data_ptr(), cos.shape[0], meta.data_ptr(), batch, width,
                                   tables.data_ptr(), tables.stride(0), block_size, k_pool.data_ptr(),
                                   v_pool.data_ptr(), stream())
    _check(st, "rope_append")


def kv_write(k, v, meta, batch, width, tables, block_size, k_pool, v_pool) -> None:
    k, v = gpu(k, "k").contiguous(), v.contiguous()
    dev = k.device
    _on(dev, v, "v", k.dtype, numel=k.numel())
    _meta(dev, meta, batch)
    _tables(tables)
    _on(dev, k_pool, "k_pool", k.dtype, True)
    _on(dev, v_pool, "v_pool", k.dtype, True)
    st = lib().specdec_kv_write(k.data_ptr(), v.data_ptr(), dtype_code(k), k.shape[1], k.shape[3], meta.data_ptr(),
                                batch, width, tables.data_ptr(), tables.stride(0), block_size, k_pool.data_ptr(),
                                v_pool.data_ptr(), stream())
    _check(st, "kv_write")


def kv_gather(k_pool, v_pool, meta, batch, tables, block_size, read_width):
    dev = gpu(k_pool, "k_pool").device
    _on(dev, v_pool, "v_pool", k_pool.dtype, True)
    _meta(dev, meta, batch)
    _tables(tables)
    n_kv, d = k_pool.shape[1], k_pool.shape[3]
    k_out = torch.empty(batch, n_kv, read_width, d, dtype=k_pool.dtype, device=k_pool.device)
    v_out = torch.empty_like(k_out)
    st = lib().specdec_kv_gather(k_pool.data_ptr(), v_pool.data_ptr(), dtype_code(k_pool), n_kv, d, meta.data_ptr(),
                                 batch, tables.data_ptr(), tables.stride(0), block_size, read_width,
                                 k_out.data_ptr(), v_out.data_ptr(), stream())
    _check(st, "kv_gather")
    return k_out, v_out


# -------------------------------------------------------------- layer glue --
def add_rmsnorm(hidden: torch.Tensor, delta: torch.Tensor | None, weight: torch.Tensor, out: torch.Tensor,
                eps: float) -> torch.Tensor:
    """hidden += delta (if given), out = RMSNorm(hidden) * weight; rows are the
    leading dims.  hidden and out must be contiguous."""
    dim = hidden.shape[-1]
    dev = gpu(hidden, "hidden").device
    _on(dev, hidden, "hidden", contiguous=True)
    _on(dev, out, "out", hidden.dtype, True, hidden.numel())
    _on(dev, weight, "weight", hidden.dtype, True, dim)
    if delta is not None:
        _on(dev, delta, "delta", hidden.dtype, True, hidden.numel())
    st = lib().specdec_add_rmsnorm(hidden.data_ptr(), ptr(delta), weight.data_ptr(), out.data_ptr(),
                                   dtype_code(hidden), hidden.numel() // dim, dim, float(eps), stream())
    _check(st, "add_rmsnorm")
    return out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    inter = gate_up.shape[-1] // 2
    dev = gpu(gate_up, "gate_up").device
    _on(dev, gate_up, "gate_up", contiguous=True)
    _on(dev, out, "out", gate_up.dtype, True, gate_up.numel() // 2)
    st = lib().specdec_silu_mul(gate_up.data_ptr(), out.data_ptr(), dtype_code(gate_up), gate_up.numel() // (2 * inter),
                                inter, stream())
    _check(st, "silu_mul")
    return out


def rms_silu_mul(gate_up: torch.Tensor, hidden: torch.Tensor, out: torch.Tensor, eps: float) -> torch.Tensor:
    """out = round(silu(round(s * gate))) * round(s * up), s = rsqrt(mean(hidden^2)
    + eps) per row: the post-attention RMSNorm finished after a gate/up
    projection of the unnormalised hidden (whose weight carries the norm
    weight in its columns).  Rows are the leading dims of all three."""
    inter, dim = gate_up.shape[-1] // 2, hidden.shape[-1]
    dev = gpu(gate_up, "gate_up").device
    _on(dev, gate_up, "gate_up", contiguous=True)
    rows = gate_up.numel() // (2 * inter)
    _on(dev, hidden, "hidden", gate_up.dtype, True, rows * dim)
    _on(dev, out, "out", gate_up.dtype, True, rows * inter)
    st = lib().specdec_rms_silu_mul(gate_up.data_ptr(), hidden.data_ptr(), out.data_ptr(), dtype_code(gate_up), rows,
                                    inter, dim, float(eps), stream())
    _check(st, "rms_silu_mul")
    return out


# --------------------------------------------------------------- attention --
class AttentionWorkspace:
    """Grow-only buffer of split-KV partials for one device.  Calls that
    share a workspace must be ordered on one stream."""

    def __init__(self, device: torch.device) -> None:
        self.device = device
        self.floats = torch.empty(0, dtype=torch.float32, device=device)

    def reserve(self, floats: int) -> None:
        if floats > self.floats.numel():
            self.floats = torch.empty(max(floats, 2 * self.floats.numel()), dtype=torch.float32, device=self.device)


def attention_workspace_floats(batch: int, width: int, n_heads: int, n_kv_heads: int, head_dim: int,
                               max_kv_len: int, split_tokens: int = 0) -> int:
    import ctypes

    floats = ctypes.c_int64()
    st = lib().specdec_attention_workspace(batch, width, n_heads, n_kv_heads, head_dim, max_kv_len, split_tokens,
                                           ctypes.byref(floats))
    _check(st, "attention_workspace")
    return floats.value


_workspaces: dict[torch.device, AttentionWorkspace] = {}


def workspace_for(device: torch.device) -> AttentionWorkspace:
    ws = _workspaces.get(device)
    if ws is None:
        ws = _workspaces[device] = AttentionWorkspace(device)
    return ws


def attention_split(batch: int, width: int, n_heads: int, n_kv_heads: int, max_kv_len: int) -> int:
    return lib().specdec_attention_split(batch, width, n_heads, n_kv_heads, max_kv_len)


DECODE_PARTS_MAX_ROWS = 16  # rows of a draft step whose attention goes through split partials
DECODE_PARTS_COUNTS = (4, 8, 16)  # partials per row and query head a launch may use
DECODE_PART_FLOATS = 4 + 64  # m, l, two unused, O


def decode_parts_count(max_kv_len: int) -> int:
    """Partials per (row, kv head) for a draft step of at most max_kv_len
    keys (the graphs' bucket, not the row's length): 4 up to 256 keys, else
    8.  Measured at the draft's shape (attention + o_proj, one row): 8 parts
    take 8.5 us at 256-384 keys against 9.3 with 4 and 9.7 with 16, and
    stay within 0.8 us of 16 parts up to 2048 keys, while 16 cost 1.3 us
    more than 8 at short contexts (idle parts, a longer fold)."""
    return 4 if max_kv_len <= 256 else 8


def decode_parts_fit(dtype: torch.dtype, batch: int, width: int, n_heads: int, n_kv_heads: int, head_dim: int,
                     block_size: int, max_kv_len: int, split_tokens: int) -> bool:
    """Shapes `rope_paged_attention_parts` + `linear_attn_parts` take: a
    latency call (split_tokens < 0) of one new bf16 token per row, at most
    16 rows, head_dim 64, block_size % 16 == 0, at most 2048 cached tokens,
    at most 16 query heads per kv head and 2048 query features."""
    return (dtype == torch.bfloat16 and width == 1 and split_tokens < 0 and 0 < batch <= DECODE_PARTS_MAX_ROWS
            and head_dim == 64 and block_size % 16 == 0 and 0 < max_kv_len <= 2048 and n_kv_heads > 0
            and n_heads % n_kv_heads == 0 and n_heads // n_kv_heads <= 16 and n_heads * head_dim <= 2048)


def decode_parts_buffer(batch: int, n_heads: int, device, nparts: int = 4) -> torch.Tensor:
    """The fp32 [batch, H, nparts, 68] buffer a draft step's attention partials go through."""
    if nparts not in DECODE_PARTS_COUNTS:
        raise ValueError(f"nparts must be one of {DECODE_PARTS_COUNTS}")
    return torch.empty(batch, n_heads, nparts, DECODE_PART_FLOATS, dtype=torch.float32, device=device)


def _parts_of(parts: torch.Tensor, dev, batch: int, n_heads: int) -> int:
    """nparts of a `decode_parts_buffer`, checked."""
    if parts.dim() != 4 or tuple(parts.shape[:2]) != (batch, n_heads) or parts.shape[3] != DECODE_PART_FLOATS:
        raise ValueError(f"parts must be fp32 [{batch}, {n_heads}, nparts, {DECODE_PART_FLOATS}]")
    _on(dev, parts, "parts", torch.float32, True)
    return parts.shape[2]


def rope_paged_attention_parts(qkv, cos, sin, k_pool, v_pool, tables, meta, batch, n_heads, n_kv_heads, head_dim,
                               block_size, scale, max_kv_len, parts: torch.Tensor,
                               norm_of: torch.Tensor | None = None, eps: float = 0.0) -> torch.Tensor:
    """A draft-style decode step (rope_paged_attention of one new token per
    row with split_tokens < 0, the same RoPE, norm and append) whose
    attention is left as split partials: nparts (parts.shape[2]) one-wave
    workgroups per (row, kv head), each writing its (m, l, O) to `parts`
    (`decode_parts_buffer`) instead of folding them in one workgroup.
    `linear_attn_parts` folds them into the attention rows (with 4 parts the
    bits rope_paged_attention produces) and projects them."""
    dev = gpu(qkv, "qkv").device
    _qkv_side(dev, qkv, cos, sin, meta, batch, 1, tables, k_pool, v_pool)
    _token_rows(qkv, batch, qkv.stride(1), (n_heads + 2 * n_kv_heads) * head_dim, "qkv")
    nparts = _parts_of(parts, dev, batch, n_heads)
    hidden_dim = 0
    if norm_of is not None:
        hidden_dim = norm_of.shape[-1]
        _on(dev, norm_of, "norm_of", qkv.dtype, True, batch * hidden_dim)
    st = lib().specdec_rope_paged_attention_parts(qkv.data_ptr(), qkv.stride(1), cos.data_ptr(), sin.data_ptr(),
                                                  ptr(norm_of), hidden_dim, float(eps), k_pool.data_ptr(),
                                                  v_pool.data_ptr(), tables.data_ptr(), tables.stride(0),
                                                  meta.data_ptr(), batch, n_heads, n_kv_heads, head_dim, block_size,
                                                  float(scale), max_kv_len, nparts, parts.data_ptr(), stream())
    _check(st, "rope_paged_attention_parts")
    return parts


def linear_attn_parts(parts: torch.Tensor, rows: int, n_heads: int, w: torch.Tensor, out: torch.Tensor,
                      accumulate: bool = False, attn_out: torch.Tensor | None = None) -> torch.Tensor:
    """`linear(attn, w, out, accumulate)` where attn [rows, H*64] are the
    attention rows a `rope_paged_attention_parts` call left as partials:
    each workgroup folds them (the attention-only kernel's arithmetic and
    order) into LDS and projects them with specdec_linear's k-split, so
    `out` gets the bits of those rows followed by linear (with 4 parts, of
    rope_paged_attention followed by linear).  `attn_out` (bf16 [rows,
    H*64]) receives the folded rows when given."""
    gpu(w, "w")
    nparts = _parts_of(parts, w.device, rows, n_heads)
    _on(w.device, out, "out", torch.bfloat16)
    if attn_out is not None:
        _on(w.device, attn_out, "attn_out", torch.bfloat16, True, rows * n_heads * 64)
    if w.dim() == 2 and w.stride(1) == 1:
        n, k, layout, w_stride = w.shape[0], w.shape[1], W_ROWS, w.stride(0)
    else:
        n, k, layout = _weight(w)
        w_stride = k
    if w.dtype != torch.bfloat16 or k != n_heads * 64:
        raise ValueError(f"w must be bf16 [N, {n_heads * 64}] (unit inner stride) or its tile_weight form")
    o2 = out.view(rows, n) if out.dim() != 2 else out
    if tuple(o2.shape) != (rows, n) or o2.stride(-1) != 1:
        raise ValueError("out must be bf16 [rows, N] with unit inner stride")
    st = lib().specdec_linear_attn_parts(parts.data_ptr(), rows, n_heads, nparts, w.data_ptr(), w_stride, layout, n,
                                         o2.data_ptr(), o2.stride(0), int(accumulate), ptr(attn_out), stream())
    _check(st, "linear_attn_parts")
    return out


def latency_split(batch: int, width: int, n_heads: int, n_kv_heads: int, max_kv_len: int) -> int:
    """A split for calls whose bits need not match any other call (the draft
    model).  With few (row, head) units: -1, one 16-wave workgroup per unit
    striding every key, so no combine kernel is launched; otherwise 0 (the
    default)."""
    units = batch * n_kv_heads * -(-(width * (n_heads // n_kv_heads)) // 16)
    return -1 if units < 64 else 0


def _qkv_side(dev, x, cos, sin, meta, batch, width, tables, k_pool, v_pool, out=None) -> None:
    """Devices and dtypes of the pointer arguments an attention or append
    launch shares: pools of the activations' dtype, fp32 RoPE tables, int32
    metadata and block tables; `out` of the activations' dtype."""
    if cos is not None:
        _on(dev, cos, "cos", torch.float32, True)
        _on(dev, sin, "sin", torch.float32, True, cos.numel())
    _meta(dev, meta, batch)
    _tables(tables)
    _on(dev, k_pool, "k_pool", x.dtype, True)
    _on(dev, v_pool, "v_pool", x.dtype, True, k_pool.numel())
    if out is not None:
        _on(dev, out, "out", x.dtype)
    if x.stride(-1) != 1:
        raise ValueError("activations need unit inner stride")
    if batch > 0 and width > 0 and x.numel() == 0:
        raise ValueError(f"no activations for batch {batch}, width {width}")


def paged_attention(q, q_token_stride, k_pool, v_pool, tables, meta, batch, width, n_heads, n_kv_heads, head_dim,
                    block_size, scale, max_kv_len, out, out_token_stride, workspace: AttentionWorkspace | None = None,
                    split_tokens: int = 0):
    _qkv_side(gpu(q, "q").device, q, None, None, meta, batch, width, tables, k_pool, v_pool, out)
    _token_rows(q, batch * width, q_token_stride, n_heads * head_dim, "q")
    _token_rows(out, batch * width, out_token_stride, n_heads * head_dim, "out")
    ws = workspace or workspace_for(q.device)
    ws.reserve(attention_workspace_floats(batch, width, n_heads, n_kv_heads, head_dim, max_kv_len, split_tokens))
    st = lib().specdec_paged_attention(q.data_ptr(), dtype_code(q), q_token_stride, k_pool.data_ptr(),
                                       v_pool.data_ptr(), tables.data_ptr(), tables.stride(0), meta.data_ptr(), batch,
                                       width, n_heads, n_kv_heads, head_dim, block_size, float(scale), max_kv_len,
                                       split_tokens, ws.floats.data_ptr(), ws.floats.numel(), out.data_ptr(),
                                       out_token_stride, stream())
    _check(st, "paged_attention")
    return out


def paged_attention_static(q, q_token_stride, k_pool, v_pool, tables, meta, batch, width, n_heads, n_kv_heads,
                           head_dim, block_size, scale, max_kv_len, out, out_token_stride, split_tokens: int = 0):
    """paged_attention with no workspace: split partials live in the
    library's own per-GPU buffer (specdec_paged_attention_static), so the
    call allocates nothing.  Raises KernelError if the call needs more
    partials than that buffer holds; calls overlapping on one GPU race."""
    _qkv_side(gpu(q, "q").device, q, None, None, meta, batch, width, tables, k_pool, v_pool, out)
    _token_rows(q, batch * width, q_token_stride, n_heads * head_dim, "q")
    _token_rows(out, batch * width, out_token_stride, n_heads * head_dim, "out")
    st = lib().specdec_paged_attention_static(q.data_ptr(), dtype_code(q), q_token_stride, k_pool.data_ptr(),
                                              v_pool.data_ptr(), tables.data_ptr(), tables.stride(0),
                                              meta.data_ptr(), batch, width, n_heads, n_kv_heads, head_dim,
                                              block_size, float(scale), max_kv_len, split_tokens, out.data_ptr(),
                                              out_token_stride, stream())
    _check(st, "paged_attention_static")
    return out


# new tokens per row up to which the attention can finish the input RMSNorm
# (every new token of a row is staged in the workgroup's LDS)
NORM_IN_ATTENTION_MAX_WIDTH = 16


def norm_in_attention(dtype: torch.dtype, block_size: int, width: int) -> bool:
    """Whether rope_paged_attention accepts `norm_of` for this call shape."""
    return dtype == torch.bfloat16 and block_size % 16 == 0 and width <= NORM_IN_ATTENTION_MAX_WIDTH


def rope_paged_attention(qkv, cos, sin, k_pool, v_pool, tables, meta, batch, width, n_heads, n_kv_heads, head_dim,
                         block_size, scale, max_kv_len, out, out_token_stride,
                         workspace: AttentionWorkspace | None = None, split_tokens: int = 0,
                         norm_of: torch.Tensor | None = None, eps: float = 0.0):
    """RoPE + paged append + verify attention in one launch (plus the split
    combine when needed).  qkv [B, T, (H + 2 Hkv) d] holds unrotated q/k/v.
    With `norm_of` (the [B, T, hidden] residual stream that qkv projects, the
    norm weight folded into the projection), each token's q/k/v are scaled by
    its row's rsqrt(mean(norm_of^2) + eps) first: the input RMSNorm finished
    after the projection (`norm_in_attention` tells which shapes allow it)."""
    dev = gpu(qkv, "qkv").device
    _qkv_side(dev, qkv, cos, sin, meta, batch, width, tables, k_pool, v_pool, out)
    _token_rows(qkv, batch * width, qkv.stride(1), (n_heads + 2 * n_kv_heads) * head_dim, "qkv")
    _token_rows(out, batch * width, out_token_stride, n_heads * head_dim, "out")
    hidden_dim = 0
    if norm_of is not None:
        if not norm_in_attention(qkv.dtype, block_size, width):
            raise ValueError(f"norm_of needs bf16, block_size % 16 == 0 and width <= {NORM_IN_ATTENTION_MAX_WIDTH}")
        hidden_dim = norm_of.shape[-1]
        _on(dev, norm_of, "norm_of", qkv.dtype, True, batch * width * hidden_dim)
    ws = workspace or workspace_for(qkv.device)
    ws.reserve(attention_workspace_floats(batch, width, n_heads, n_kv_heads, head_dim, max_kv_len, split_tokens))
    st = lib().specdec_rope_paged_attention(qkv.data_ptr(), dtype_code(qkv), qkv.stride(1), cos.data_ptr(),
                                            sin.data_ptr(), ptr(norm_of), hidden_dim, float(eps), k_pool.data_ptr(),
                                            v_pool.data_ptr(), tables.data_ptr(),
                                            tables.stride(0), meta.data_ptr(), batch, width, n_heads, n_kv_heads,
                                            head_dim, block_size, float(scale), max_kv_len, split_tokens,
                                            ws.floats.data_ptr(), ws.floats.numel(), out.data_ptr(), out_token_stride,
                                            stream())
    _check(st, "rope_paged_attention")
    return out
