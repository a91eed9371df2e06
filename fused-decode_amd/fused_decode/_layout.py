"""Row layouts shared by the row-wise kernels (norms, RoPE, SwiGLU).

A tensor is seen as a grid of rows over its last dimension, with up to three
leading dimensions of arbitrary (including zero) strides plus a column stride:
the contract of RowLayout in the reference (src/fused_decode/kernels.py:26-70).

Unlike the reference, the operands of one launch are laid out *jointly*: size-1
dims are dropped and adjacent leading dims are merged only where every operand
allows it, so all operands always share one row grid. A layout that cannot be
expressed (more than three unmergeable leading dims) is handled explicitly: an
input is copied to a contiguous tensor, and an output is computed into a
contiguous temporary that is then copied back into the caller's tensor. The
reference's ``.contiguous()`` on such an ``out`` would silently drop the write
(kernels.py:47-51). PyTorch tensors never carry negative strides, so the
reference's negative-stride branch has no counterpart here.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ._lib import FdRows


@dataclass
class Operand:
    tensor: torch.Tensor      # what the kernel reads or writes
    target: torch.Tensor | None  # caller's output to copy back into, if a temporary is used
    rows: FdRows


def _plan(shape: tuple[int, ...], strides_list: list[tuple[int, ...]]):
    """Merged leading dims: list of (size, [stride per operand])."""
    lead = [i for i in range(len(shape) - 1) if shape[i] != 1]
    dims: list[tuple[int, list[int]]] = []
    for i in lead:
        if dims:
            size, strides = dims[-1]
            # merge with previous when previous stride == this stride * this size
            if all(strides[k] == strides_list[k][i] * shape[i] for k in range(len(strides_list))):
                dims[-1] = (size * shape[i], [strides_list[k][i] for k in range(len(strides_list))])
                continue
        dims.append((shape[i], [st[i] for st in strides_list]))
    return dims


def _rows_from(dims, k: int, col: int, n: int) -> FdRows:
    sizes = [1, 1, 1]
    strides = [0, 0, 0]
    off = 3 - len(dims)
    for j, (size, st) in enumerate(dims):
        sizes[off + j] = size
        strides[off + j] = st[k]
    return FdRows(sizes[0], sizes[1], sizes[2], strides[0], strides[1], strides[2], col, n)


def contiguous_strides(shape) -> tuple[int, ...]:
    """Strides of a dense row-major tensor of ``shape``."""
    out, step = [], 1
    for size in reversed(tuple(shape)):
        out.append(step)
        step *= max(int(size), 1)
    return tuple(reversed(out))


def plan_rows(shape, strides_list: list[tuple[int, ...]]) -> list[bytes] | None:
    """Packed ``fd_rows`` (bytes, as the C ABI takes them) for operands that share
    ``shape``, one per stride tuple, or None when their common row grid needs
    more than three leading dims (the caller then stages through contiguous
    copies). Depends on shapes and strides only, so it can be computed once per
    argument signature."""
    shape = tuple(shape)
    n = shape[-1]
    if n and all(st == strides_list[0] for st in strides_list) and \
            tuple(strides_list[0]) == contiguous_strides(shape):
        rows = FdRows(1, 1, _numel(shape) // n, 0, 0, n, 1, n)
        return [bytes(rows)] * len(strides_list)
    dims = _plan(shape, [tuple(st) for st in strides_list])
    if len(dims) > 3:
        return None
    return [bytes(_rows_from(dims, k, int(st[-1]) if n != 1 else 1, n)) for k, st in enumerate(strides_list)]


def _numel(shape) -> int:
    total = 1
    for s in shape:
        total *= int(s)
    return total


def joint_layout(inputs: list[torch.Tensor], outputs: list[torch.Tensor]) -> tuple[list[Operand], list[Operand]]:
    """Row layouts for operands of one shape (broadcast inputs already expanded)."""
    shape = inputs[0].shape
    if len(shape) == 0:
        raise ValueError("expected a tensor with a last dimension")
    n = shape[-1]
    if n and all(t.is_contiguous() for t in inputs) and all(t.is_contiguous() for t in outputs):
        # every operand is the same dense [rows, n] block: one shared layout
        rows = FdRows(1, 1, inputs[0].numel() // n, 0, 0, n, 1, n)
        return [Operand(t, None, rows) for t in inputs], [Operand(t, None, rows) for t in outputs]
    shape = tuple(shape)
    ins = list(inputs)
    outs: list[torch.Tensor] = list(outputs)
    targets: list[torch.Tensor | None] = [None] * len(outs)
    allt = ins + outs
    dims = _plan(shape, [tuple(t.stride()) for t in allt])
    if len(dims) > 3:
        ins = [t.contiguous() for t in ins]
        for i, t in enumerate(outs):
            if not t.is_contiguous():
                targets[i] = t if targets[i] is None else targets[i]
                outs[i] = torch.empty(shape, dtype=t.dtype, device=t.device)
        allt = ins + outs
        dims = _plan(shape, [tuple(t.stride()) for t in allt])
    ops = []
    for k, t in enumerate(allt):
        col = int(t.stride(-1)) if n != 1 else 1
        ops.append(Operand(t, None, _rows_from(dims, k, col, n)))
    for i in range(len(outs)):
        ops[len(ins) + i].target = targets[i]
    return ops[: len(ins)], ops[len(ins):]


def finish(outputs: list[Operand]) -> None:
    """Copy temporaries back into the caller's output tensors."""
    for op in outputs:
        if op.target is not None:
            op.target.copy_(op.tensor)
