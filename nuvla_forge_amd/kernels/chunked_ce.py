"""Memory-bounded cross entropy for the reasoning head, on MI355X MFMA.

Drop-in for ``nuvla_forge/kernels/chunked_ce.py``: the same
``_ChunkedCrossEntropy`` autograd Function (``forward(ctx, hidden, lm_weight,
targets, chunk_size, ignore_index, force_reference) -> loss``; ``backward``
returns 6 values, chunked_ce.py:120-182) and the same public
``chunked_cross_entropy(hidden, lm_weight, targets, chunk_size=1024,
ignore_index=-100, force_reference=False)`` (chunked_ce.py:185-208).

The device path is two calls.  ``nf_ce_fwd`` compacts the valid rows on the
device and, ``chunk_size`` of them at a time, forms their logits once on
bf16 (or fp32) MFMA and keeps them as ``exp(logit - target logit)`` in both
layouts the gradient products read, with a per-row factor (from an fp32
log-sum-exp over per-tile statistics) that makes them ``(softmax - onehot) /
n``; it runs the gradient products of every chunk but the last, and the loss
comes out.  ``nf_ce_bwd`` runs the last
chunk's products with ``grad_output`` known and writes both gradients scaled,
in each input's dtype.  The reference forms fp32 gradients in the forward
pass and scales and casts them in the backward; the results are the same.
The valid-token count stays on the device, so a device call makes no host
synchronisation at all (the reference's ``.item()`` at chunked_ce.py:126 is
gone): targets outside ``[0, V)`` that are not ``ignore_index`` are counted
on the device and treated as ignored.  Setting ``VALIDATE_TARGETS = True``
opts into raising ``ValueError`` for them instead, at the price of one
device-to-host read per call (skipped while a graph is being captured).

Host tensors (and ``force_reference=True``) run the reference's own row-chunk
loop in ATen (chunked_ce.py:133-167 with ``_ce_chunk_torch``, :101-117).

``chunk_size`` bounds memory by what the reference's row-chunk loop holds at
the same setting: in bf16 a chunk's probabilities and the fp32 dW
accumulator together stay within the bytes of its fp32 [chunk_size, V]
logits tile plus its fp32 [V, D] dW accumulator (up to 256-row rounding).
Where the probabilities of every row fit that, one chunk takes them all with
no accumulator (held once, or for D >= 2048 in both layouts the gradient
products read when those fit); otherwise chunks of 2 * chunk_size valid
rows are held once (the dW product reads them transposed) beside the
accumulator.  fp32 holds chunks of chunk_size rows in both layouts.  Fewer
chunks are faster (no passes over the accumulator); results do not depend
on chunk_size beyond fp rounding.

Element types: under bf16 autocast for the device the products run in bf16
(MFMA, fp32 accumulation) whatever the input types, as the reference's
autocast-ed ``F.linear`` and ``@`` do; otherwise bf16 inputs run bf16 MFMA,
fp32 inputs fp32 MFMA, and mixed or fp16 inputs are widened to fp32.
"""

from __future__ import annotations

import torch

from .. import _lib
from .utils import check_devices, device_of, use_fused

# Opt-in: raise ValueError for targets outside [0, V) that are not
# ignore_index.  The check reads one device int back to the host (a
# synchronisation), so it is off by default, when such rows count as ignored;
# it is skipped while a stream is being captured into a graph.
VALIDATE_TARGETS = False


def chunk_rows_for(chunk_size: int) -> int:
    """Rows per chunk the device path is asked for (the library rounds up to 256)."""
    if int(chunk_size) <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk_size}")
    return int(chunk_size)


def _compute_dtype(hidden: torch.Tensor, lm_weight: torch.Tensor) -> torch.dtype:
    """bf16 under bf16 autocast for the device (what F.linear would compute in,
    even for the fp32 residual stream and fp32 lm_head of the reasoning head),
    else the inputs' shared bf16 / fp32 type, else fp32."""
    dev = hidden.device.type
    if torch.is_autocast_enabled(dev) and torch.get_autocast_dtype(dev) == torch.bfloat16:
        return torch.bfloat16
    hd, wd = hidden.dtype, lm_weight.dtype
    if hd == wd and hd in (torch.bfloat16, torch.float32):
        return hd
    return torch.float32


def _ce_chunk_torch(logits, targets, ignore_index, inv_count):
    """One row chunk in ATen: (sum of row losses * inv, (softmax - onehot) * inv).

    Same quantities as the reference's CPU chunk path (chunked_ce.py:101-117);
    ignored rows get zero loss and a zero gradient row.
    """
    logits = logits.float()
    keep = (targets != ignore_index).to(logits.dtype)
    rows = torch.arange(targets.shape[0], device=logits.device)
    cols = torch.where(targets != ignore_index, targets, torch.zeros_like(targets))
    lse = torch.logsumexp(logits, dim=-1)
    loss = (lse - logits[rows, cols]) * keep
    grad = torch.exp(logits - lse.unsqueeze(1))
    grad[rows, cols] -= 1.0
    grad *= keep.unsqueeze(1)
    return loss.sum() * inv_count, grad * inv_count


def _forward_eager(hidden, lm_weight, targets, chunk_size, ignore_index):
    """The reference's row-chunk loop in ATen (``force_reference=True``)."""
    m = hidden.shape[0]
    n_valid = int((targets != ignore_index).sum().item())
    inv_count = 1.0 / max(n_valid, 1)
    loss_total = hidden.new_zeros((), dtype=torch.float32)
    d_hidden = torch.zeros_like(hidden, dtype=torch.float32)
    d_weight = torch.zeros_like(lm_weight, dtype=torch.float32)
    w = lm_weight.float()
    for start in range(0, m, chunk_size):
        stop = min(start + chunk_size, m)
        h_chunk = hidden[start:stop].float()
        logits = h_chunk @ w.T
        chunk_loss, dlogits = _ce_chunk_torch(logits, targets[start:stop], ignore_index, inv_count)
        loss_total = loss_total + chunk_loss
        d_hidden[start:stop] = dlogits @ w
        d_weight += dlogits.T @ h_chunk
    return loss_total, d_hidden, d_weight


class _DeviceCall:
    """What the two device calls share besides the state tensor: the shape
    and the compute type.  The state (nf_ce_fwd's output, nf_ce_bwd's input)
    travels through ``ctx.save_for_backward``, so autograd frees it once the
    backward has run."""

    def __init__(self, m, d, v, chunk_rows, cdt):
        self.m, self.d, self.v, self.chunk_rows, self.cdt = m, d, v, chunk_rows, cdt
        self.code = _lib.dtype_code(cdt)


def _forward_hip(hidden, lm_weight, targets, chunk_size, ignore_index):
    """(loss, call record, state) for ``_backward_hip``; state is None when
    there are no rows."""
    m, d = hidden.shape
    v = lm_weight.shape[0]
    cdt = _compute_dtype(hidden, lm_weight)
    call = _DeviceCall(m, d, v, chunk_rows_for(chunk_size), cdt)
    dev = hidden.device
    loss = torch.empty((), dtype=torch.float32, device=dev)
    if m == 0:
        return loss.zero_(), call, None
    h = hidden.to(cdt).contiguous()
    w = lm_weight.to(cdt).contiguous()
    tg = targets.to(torch.int64).contiguous()
    validate = VALIDATE_TARGETS and not torch.cuda.is_current_stream_capturing()
    bad = torch.empty(1, dtype=torch.int32, device=dev) if validate else None
    L = _lib.lib()
    shape = (m, d, v, call.chunk_rows, call.code)
    st_bytes = L.nf_ce_state_bytes(*shape)
    ws_bytes = L.nf_ce_fwd_workspace(*shape)
    if not st_bytes or not ws_bytes:
        raise ValueError(f"chunked_cross_entropy: shape M={m} D={d} V={v} is beyond the kernels")
    state = torch.empty(st_bytes, dtype=torch.uint8, device=dev)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    with device_of(hidden):
        _lib.check(
            L.nf_ce_fwd(h.data_ptr(), w.data_ptr(), tg.data_ptr(), m, d, v, int(ignore_index),
                        call.chunk_rows, call.code, loss.data_ptr(), _lib.ptr(bad),
                        state.data_ptr(), st_bytes, ws.data_ptr(), ws_bytes,
                        _lib.stream_of(hidden)),
            "nf_ce_fwd",
        )
    if validate:
        nbad = int(bad.item())  # the opt-in check's one host synchronisation
        if nbad:
            raise ValueError(f"chunked_cross_entropy: {nbad} target(s) outside [0, {v}) "
                             f"and not ignore_index={ignore_index}")
    return loss, call, state


def _backward_hip(call, state, grad_output, hidden_dtype, weight_dtype, dev):
    """(grad_output * dL/dhidden, grad_output * dL/dweight) in the inputs' dtypes."""
    check_devices("chunked_cross_entropy backward", "the forward's hidden",
                  {"grad_output": grad_output}, device=dev)
    m, d, v = call.m, call.d, call.v
    dh = torch.empty((m, d), dtype=hidden_dtype, device=dev)
    dw = torch.empty((v, d), dtype=weight_dtype, device=dev)
    if m == 0:
        return dh, dw.zero_()
    g = grad_output.to(torch.float32).contiguous()
    L = _lib.lib()
    ws_bytes = L.nf_ce_bwd_workspace(m, d, v, call.chunk_rows, call.code)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    with device_of(dh):
        _lib.check(
            L.nf_ce_bwd(m, d, v, call.chunk_rows, call.code, state.data_ptr(),
                        state.numel(), g.data_ptr(), dh.data_ptr(), _lib.dtype_code(dh),
                        dw.data_ptr(), _lib.dtype_code(dw), ws.data_ptr(), ws_bytes,
                        _lib.stream_of(dh)),
            "nf_ce_bwd",
        )
    return dh, dw


class _ChunkedCrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, lm_weight, targets, chunk_size, ignore_index, force_reference):
        if hidden.dim() != 2 or lm_weight.dim() != 2 or hidden.shape[1] != lm_weight.shape[1]:
            raise ValueError(f"hidden [M, D] and lm_weight [V, D] expected, got "
                             f"{tuple(hidden.shape)} and {tuple(lm_weight.shape)}")
        if targets.shape != (hidden.shape[0],):
            raise ValueError(f"targets must be [M={hidden.shape[0]}], got {tuple(targets.shape)}")
        check_devices("chunked_cross_entropy", "hidden",
                      dict(hidden=hidden, lm_weight=lm_weight, targets=targets))
        ctx.hidden_dtype = hidden.dtype
        ctx.weight_dtype = lm_weight.dtype
        # the reference's rule (chunked_ce.py:133): the eager chunk loop for
        # force_reference and for host tensors, the device kernels otherwise
        ctx.eager = not use_fused(hidden, "chunked_cross_entropy", force_reference)
        if ctx.eager:
            loss, d_hidden, d_weight = _forward_eager(hidden, lm_weight, targets, chunk_size,
                                                      ignore_index)
            ctx.save_for_backward(d_hidden, d_weight)
            return loss
        loss, ctx.call, state = _forward_hip(hidden, lm_weight, targets, chunk_size,
                                             ignore_index)
        # through save_for_backward, not a ctx attribute: autograd releases
        # the state (hundreds of MB at the BASELINE shape) after the backward
        ctx.save_for_backward(state)
        ctx.device = hidden.device
        return loss

    @staticmethod
    def backward(ctx, grad_output):
        if ctx.eager:
            d_hidden, d_weight = ctx.saved_tensors
            g = grad_output
            return ((d_hidden * g).to(ctx.hidden_dtype), (d_weight * g).to(ctx.weight_dtype),
                    None, None, None, None)
        (state,) = ctx.saved_tensors
        dh, dw = _backward_hip(ctx.call, state, grad_output, ctx.hidden_dtype,
                               ctx.weight_dtype, ctx.device)
        return dh, dw, None, None, None, None


def chunked_cross_entropy(
    hidden: torch.Tensor,
    lm_weight: torch.Tensor,
    targets: torch.Tensor,
    chunk_size: int = 1024,
    ignore_index: int = -100,
    force_reference: bool = False,
) -> torch.Tensor:
    """Mean cross entropy over ``hidden @ lm_weight.T`` without a full logit tensor.

    Args:
        hidden: [M, D] pre-projection hidden states.
        lm_weight: [V, D] output embedding.
        targets: [M] int64 class indices, ``ignore_index`` to mask.
        chunk_size: memory budget: the bytes of the reference's fp32
            [chunk_size, V] logits tile plus its fp32 [V, D] dW accumulator.
        ignore_index: target value that contributes no loss and no gradient.
        force_reference: run the reference's eager row-chunk loop instead.

    Returns:
        Scalar fp32 loss, mean-reduced over non-ignored tokens (0 if none).

    Host tensors run the reference's eager row-chunk loop, as in the reference.
    """
    return _ChunkedCrossEntropy.apply(hidden, lm_weight, targets, chunk_size, ignore_index,
                                      force_reference)
