"""Host-side helpers of special_attentions/utils/tools.py that the reference's processor
modules import (`from special_attentions.utils.tools import preserve_rng_state, timeit`).

`timeit` follows tools.py:3-12 and `preserve_rng_state` tools.py:162-181. The plotting
helpers of that file (`visualize_head_seq`, `analyze_and_visualize`) draw matplotlib figures
of recorded tensors and sparsity logs; they are not part of the attention path and are not
provided.
"""
from __future__ import annotations

import functools
import time

import torch


def timeit(func):
    """Decorator: runs `func` between two device synchronisations and prints its wall time,
    "<name> execution took <ms>ms" (tools.py:3-12)."""

    @functools.wraps(func)
    def timed(*args, **kwargs):
        if torch.cuda.is_available():
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = func(*args, **kwargs)
        if torch.cuda.is_available():
            torch.cuda.synchronize()
        print(f"{func.__name__} execution took {(time.perf_counter() - t0) * 1e3:.4f}ms")
        return out

    return timed


class rng_state_preserved:
    """Context manager: the CPU generator state and every visible GPU's generator state are
    restored on exit, also when the body raises."""

    def __enter__(self):
        self.cpu = torch.get_rng_state()
        self.cuda = [torch.cuda.get_rng_state(d) for d in range(torch.cuda.device_count())] \
            if torch.cuda.is_available() else []
        return self

    def __exit__(self, *exc):
        torch.set_rng_state(self.cpu)
        for d, s in enumerate(self.cuda):
            torch.cuda.set_rng_state(s, d)
        return False


def preserve_rng_state(func):
    """Decorator form of `rng_state_preserved` (tools.py:162-181): random draws inside `func`
    leave the callers' generator states as they were."""

    @functools.wraps(func)
    def guarded(*args, **kwargs):
        with rng_state_preserved():
            return func(*args, **kwargs)

    return guarded
