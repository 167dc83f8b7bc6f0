"""torch.library registrations of this package's C-ABI calls (namespace
`uttt_hip`), each with a fake implementation that gives its outputs' shapes
and dtypes, so that torch.compile traces the drop-in ops into its graph
instead of breaking the graph at every kernel call.

`traced_op(name, fake)` registers a function as torch.ops.uttt_hip.<name>
and returns a wrapper that calls the registered op while torch.compile
traces, and the function itself otherwise (eager calls skip the dispatcher).
"""
from __future__ import annotations

import functools

import torch


def traced_op(name, fake, mutates_args=()):
    def deco(fn):
        op = torch.library.custom_op(f"uttt_hip::{name}", fn, mutates_args=mutates_args)
        op.register_fake(fake)

        @functools.wraps(fn)
        def call(*args, **kwargs):
            if torch.compiler.is_compiling():
                return op(*args, **kwargs)
            return fn(*args, **kwargs)

        call.op = op
        return call

    return deco


def none_if_empty(t):
    """Optional outputs travel through the ops as 0-element tensors."""
    return None if t is None or t.numel() == 0 else t


def empty_like_dev(ref, *shape, dtype=None):
    return ref.new_empty(shape, dtype=ref.dtype if dtype is None else dtype)
