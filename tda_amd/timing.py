"""Per-kernel durations of C-ABI calls (tda_time_next_call in include/tda.h).

The library records the caller's HIP events on the call's own stream before its first kernel
launch and after each launch, so each kernel's duration is the time between two consecutive
events, measured on the stream the kernel ran on.  Arming is per host thread and covers the
next tda_fwd / tda_fwd_noalloc / tda_bwd call made by that thread.

    timer = LaunchTimer(calls=100)
    for _ in range(100):
        timer.arm()
        ops.forward(...)          # exactly one C-ABI call after arm()
        timer.collect()
    torch.cuda.synchronize()
    timer.mean_us()               # {"key_prep": ..., "fwd_screen": ..., ...}
"""
from __future__ import annotations

import ctypes

import torch

from . import _abi


class LaunchTimer:
    """Events for `calls` timed C-ABI calls of at most `max_launches` kernel launches each."""

    def __init__(self, calls: int, max_launches: int = 8, device=None):
        self.lib = _abi.load()
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.n = max_launches + 1
        stream = torch.cuda.current_stream(self.device)
        self.events = [[torch.cuda.Event(enable_timing=True) for _ in range(self.n)] for _ in range(calls)]
        for evs in self.events:  # torch creates the HIP event at its first record
            for e in evs:
                e.record(stream)
        torch.cuda.synchronize(self.device)
        self.handles = [(ctypes.c_void_p * self.n)(*[e.cuda_event for e in evs]) for evs in self.events]
        self.calls: list[list[str]] = []  # launch names of each collected call

    def arm(self) -> None:
        k = len(self.calls)
        if k >= len(self.events):
            raise RuntimeError(f"LaunchTimer: all {len(self.events)} event sets used")
        _abi.check(self.lib.tda_time_next_call(self.handles[k], self.n), "tda_time_next_call")

    def collect(self) -> list[str]:
        """Record the launches of the call just made (after arm())."""
        count = self.lib.tda_timed_launches()
        names = []
        for j in range(min(count, self.n - 1)):
            s = self.lib.tda_timed_launch_name(j)
            names.append(s.decode() if s else f"launch{j}")
        if count > self.n - 1:
            raise RuntimeError(f"LaunchTimer: the call made {count} launches, more than {self.n - 1}")
        self.calls.append(names)
        return names

    def per_call_us(self) -> list[list[float]]:
        """Duration of each launch of each collected call, in microseconds (synchronises)."""
        torch.cuda.synchronize(self.device)
        out = []
        for evs, names in zip(self.events, self.calls):
            out.append([evs[j].elapsed_time(evs[j + 1]) * 1e3 for j in range(len(names))])
        return out

    def mean_us(self) -> dict[str, float]:
        """Average duration of each kernel family over the collected calls (a family launched
        more than once in a call is summed within the call)."""
        per = self.per_call_us()
        tot: dict[str, float] = {}
        for names, us in zip(self.calls, per):
            for name, t in zip(names, us):
                tot[name] = tot.get(name, 0.0) + t
        k = max(len(self.calls), 1)
        return {name: t / k for name, t in tot.items()}

    def total_us(self) -> float:
        """Average time from the first event to the last of a call (all its launches)."""
        torch.cuda.synchronize(self.device)
        ts = [evs[0].elapsed_time(evs[len(names)]) * 1e3 for evs, names in zip(self.events, self.calls) if names]
        return sum(ts) / max(len(ts), 1)
