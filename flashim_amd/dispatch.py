"""Standalone op dispatch for this package, exposing the call surface of FlashIM's op plugin API
(``flashim/ops/_registry.py:164-428``: ``register`` / ``get`` / ``bind`` / ``explain`` / ``supports`` and the
``FLASHIM_OPS`` override grammar) so code written against ``flashim.ops`` runs unchanged on ``flashim_amd.ops``.

The table is built for a backend that has no fallback. An op here holds only HIP impls; a call picks the first impl,
in (priority, narrowest device spec, registration) order, whose device and features match the arguments' platform and whose ``accepts``
(on the trailing weight operands) and ``when`` (on all arguments) predicates pass. When none does, the call raises
``NotImplementedError`` with every impl's reason: this package never computes a result anywhere but on its kernels.
Inside FlashIM (:mod:`flashim_amd.plugin`) the same impls are registered on FlashIM's own ops, whose torch
references are then the fallback.

Each eager call runs inside a profiler range named ``flashim::<op>[<impl>]`` (a ROCTX range when
``FLASHIM_AMD_MARKERS=1`` so ``rocprofv3 --marker-trace`` shows it, else a ``torch.profiler`` range while that
profiler records) and counts toward :func:`call_counts`; the first call of each (op, impl) pair is logged at DEBUG.
Under ``torch.compile`` the selection is traced like any Python and none of the bookkeeping runs.
"""

from __future__ import annotations

import contextlib
import logging
import os
from collections import Counter
from collections.abc import Callable, Iterable
from dataclasses import dataclass, fields, is_dataclass

import torch

from flashim_amd.platforms import Feature, Platform, platform_for

logger = logging.getLogger("flashim_amd.ops")

OPS: dict[str, "Op"] = {}
_MARKERS = os.environ.get("FLASHIM_AMD_MARKERS", "0") == "1"


@dataclass(frozen=True)
class DeviceSpec:
    """Where an impl may run: a platform dispatch key (``"rocm"``, ``"cuda"``, ``"cpu"``, or ``"*"``), optionally a
    capability range (only meaningful for platforms that report one)."""

    type: str
    min_capability: tuple[int, int] | None = None
    max_capability: tuple[int, int] | None = None

    def matches(self, platform: Platform) -> bool:
        if self.type != "*" and self.type != platform.device_type:
            return False
        cap = platform.capability
        lo_ok = self.min_capability is None or (cap is not None and cap >= self.min_capability)
        hi_ok = self.max_capability is None or (cap is not None and cap <= self.max_capability)
        return lo_ok and hi_ok

    @property
    def span(self) -> float:
        """How many capability versions the spec covers (major * 100 + minor, open ends at 0.0 and 99.99; ``"*"`` is
        unbounded). Among impls of equal priority the narrower spec, the more specialized impl, is tried first."""
        if self.type == "*":
            return float("inf")
        lo = self.min_capability or (0, 0)
        hi = self.max_capability or (99, 99)
        return float((hi[0] * 100 + hi[1]) - (lo[0] * 100 + lo[1]))


@dataclass(frozen=True)
class _Entry:
    name: str
    fn: Callable
    device: DeviceSpec
    requires: frozenset
    priority: int
    when: Callable[..., bool] | None
    prepare: Callable[..., tuple] | None
    accepts: Callable[..., bool] | None
    seq: int

    def why_not(self, platform: Platform, args: tuple, kwargs: dict, weights: int,
                check_accepts: bool = True) -> str | None:
        """``None`` when this impl applies to the call, else the reason it does not."""
        if not self.device.matches(platform):
            return f"registered for {self.device.type}, call is on {platform.device_type}"
        missing = [f.value for f in self.requires if not platform.supports(f)]
        if missing:
            return "platform lacks " + ",".join(sorted(missing))
        if check_accepts and self.accepts is not None and not self.accepts(*args[len(args) - weights:]):
            return "accepts() refused the weights"
        if self.when is not None and not self.when(*args, **kwargs):
            return "when() refused the arguments"
        return None


class _Overrides:
    """``FLASHIM_OPS``: comma-separated ``-op`` (switch the op off: calls raise) and ``op:impl`` (pin an impl)."""

    def __init__(self) -> None:
        self.off: frozenset[str] = frozenset()
        self.pins: dict[str, str] = {}

    def parse(self, spec: str | None) -> None:
        off, pins = set(), {}
        for token in filter(None, (t.strip() for t in (spec or "").split(","))):
            if token.startswith("+"):
                continue
            if token.startswith("-"):
                off.add(token[1:])
            elif ":" in token:
                op, impl = token.split(":", 1)
                pins[op] = impl
            else:
                raise ValueError(f"FLASHIM_OPS: cannot parse {token!r} (use -op or op:impl)")
        self.off, self.pins = frozenset(off), pins


_OVERRIDES = _Overrides()


def configure(spec: str | None) -> None:
    """Replace the active overrides with ``spec`` (the ``FLASHIM_OPS`` grammar)."""
    _OVERRIDES.parse(spec)


configure(os.environ.get("FLASHIM_OPS"))


def _device_of(values: Iterable) -> torch.device | None:
    """The device of the first tensor among ``values`` (looking into containers and dataclasses)."""
    for v in values:
        if isinstance(v, torch.Tensor):
            return v.device
        if is_dataclass(v) and not isinstance(v, type):
            v = tuple(getattr(v, f.name) for f in fields(v))
        if isinstance(v, (tuple, list)):
            found = _device_of(v)
            if found is not None:
                return found
    return None


def _range(name: str):
    if _MARKERS and torch.cuda.is_available():
        return torch.cuda.nvtx.range(name)  # ROCTX on ROCm builds of torch
    if torch.autograd._profiler_enabled():
        return torch.profiler.record_function(name)
    return contextlib.nullcontext()


class Op:
    """One op: a name, the number of trailing weight operands that ``bind`` fixes, and its impls."""

    def __init__(self, name: str, *, weights: int = 0) -> None:
        if name in OPS:
            raise ValueError(f"op {name!r} is already declared")
        self.name, self.weights = name, weights
        self._entries: list[_Entry] = []
        self.calls: Counter[str] = Counter()
        OPS[name] = self

    @property
    def impls(self) -> list[_Entry]:
        return list(self._entries)

    def register(self, name: str, *, device: DeviceSpec, requires: Iterable[Feature] = (), priority: int = 0,
                 when: Callable[..., bool] | None = None, prepare: Callable[..., tuple] | None = None,
                 accepts: Callable[..., bool] | None = None) -> Callable[[Callable], Callable]:
        """Decorator adding ``fn`` as impl ``name``. Negative priority: used only when pinned. ``prepare`` packs the
        weight operands once per :meth:`bind`; ``accepts`` judges them."""
        if any(e.name == name for e in self._entries):
            raise ValueError(f"op {self.name!r} already has an impl named {name!r}")
        if (prepare is not None or accepts is not None) and self.weights == 0:
            raise ValueError(f"op {self.name!r} has no weight operands for prepare/accepts")

        def add(fn: Callable) -> Callable:
            self._entries.append(_Entry(name, fn, device, frozenset(requires), priority, when, prepare, accepts,
                                        len(self._entries)))
            self._entries.sort(key=lambda e: (-e.priority, e.device.span, e.seq))
            return fn

        return add

    def _entry(self, name: str) -> _Entry:
        for e in self._entries:
            if e.name == name:
                return e
        raise ValueError(f"op {self.name!r} has no impl {name!r}; it has {[e.name for e in self._entries]}")

    def _platform(self, args: tuple, kwargs: dict) -> Platform:
        return platform_for(_device_of(args) or _device_of(kwargs.values()) or torch.device("cpu"))

    def _pick(self, args: tuple, kwargs: dict, pin: str | None = None,
              accepted: dict[str, bool] | None = None) -> _Entry | None:
        if self.name in _OVERRIDES.off:
            return None
        pin = _OVERRIDES.pins.get(self.name, pin)
        platform = self._platform(args, kwargs)
        pool = [self._entry(pin)] if pin is not None else [e for e in self._entries if e.priority >= 0]
        for e in pool:
            if e.accepts is not None and accepted is not None:  # a bound op judges its weights once per impl
                if e.name not in accepted:
                    accepted[e.name] = bool(e.accepts(*args[len(args) - self.weights:]))
                if accepted[e.name] and e.why_not(platform, args, kwargs, self.weights, check_accepts=False) is None:
                    return e
            elif e.why_not(platform, args, kwargs, self.weights) is None:
                return e
        return None

    def explain(self, *args, **kwargs) -> dict[str, str]:
        """``{impl name: "selected" | reason}`` for this call."""
        platform = self._platform(args, kwargs)
        chosen = self._pick(args, kwargs)
        report = {}
        for e in self._entries:
            if chosen is not None and e.name == chosen.name:
                report[e.name] = "selected"
            elif self.name in _OVERRIDES.off:
                report[e.name] = "switched off by FLASHIM_OPS"
            else:
                report[e.name] = e.why_not(platform, args, kwargs, self.weights) or (
                    "opt-in (negative priority): pin it" if e.priority < 0 else "a higher-priority impl applies")
        return report

    def supports(self, *args, **kwargs) -> bool:
        return self._pick(args, kwargs) is not None

    def _refuse(self, args: tuple, kwargs: dict):
        reasons = "; ".join(f"{k}: {v}" for k, v in self.explain(*args, **kwargs).items()) or "no impl registered"
        raise NotImplementedError(f"op {self.name!r}: no HIP impl applies to these arguments ({reasons}); "
                                  "flashim_amd has no torch fallback")

    def _run(self, entry: _Entry | None, args: tuple, kwargs: dict, prepared: tuple | None = None):
        if entry is None:
            self._refuse(args, kwargs)
        call_args = args
        if entry.prepare is not None:
            split = len(args) - self.weights
            call_args = args[:split] + (prepared if prepared is not None else tuple(entry.prepare(*args[split:])))
        if torch.compiler.is_compiling():
            return entry.fn(*call_args, **kwargs)
        if entry.name not in self.calls:
            logger.debug("op %s -> %s", self.name, entry.name)
        self.calls[entry.name] += 1
        with _range(f"flashim::{self.name}[{entry.name}]"):
            return entry.fn(*call_args, **kwargs)

    def __call__(self, *args, **kwargs):
        return self._run(self._pick(args, kwargs), args, kwargs)

    def get(self, name: str | None) -> Callable:
        """This op with impl ``name`` pinned (``None``: the op itself). A pinned impl that does not apply raises."""
        if name is None:
            return self
        self._entry(name)
        return lambda *args, **kwargs: self._run(self._pick(args, kwargs, pin=name), args, kwargs)

    def bind(self, *weights, impl: str | None = None) -> BoundOp:
        if len(weights) != self.weights:
            raise ValueError(f"op {self.name!r} takes {self.weights} weight operands, got {len(weights)}")
        if impl is not None:
            self._entry(impl)
        return BoundOp(self, weights, impl)

    def __repr__(self) -> str:
        return f"Op({self.name}: {', '.join(e.name for e in self._entries) or 'no impls'})"


class BoundOp:
    """An op with its trailing weight operands fixed; each impl's ``prepare`` runs at most once."""

    def __init__(self, op: Op, weights: tuple, pin: str | None) -> None:
        self.op, self.weights, self.pin = op, weights, pin
        self._packed: dict[str, tuple] = {}
        self._accepted: dict[str, bool] = {}

    def _usable(self) -> list[_Entry]:
        platform = platform_for(_device_of(self.weights) or torch.device("cpu"))
        out = []
        for e in self.op.impls:
            if self.pin is not None and e.name != self.pin:
                continue
            if self.pin is None and e.priority < 0:
                continue
            if not e.device.matches(platform) or not platform.supports(*e.requires):
                continue
            if e.accepts is not None and not e.accepts(*self.weights):
                continue
            out.append(e)
        return out

    @property
    def available(self) -> list[str]:
        return [e.name for e in self._usable()]

    @property
    def primary(self) -> str | None:
        usable = self.available
        return usable[0] if usable else None

    def _prepared(self, e: _Entry) -> tuple | None:
        if e.prepare is None:
            return None
        if e.name not in self._packed:
            self._packed[e.name] = tuple(e.prepare(*self.weights))
        return self._packed[e.name]

    def warmup(self) -> BoundOp:
        for e in self._usable():
            self._prepared(e)
        return self

    def __call__(self, *args, **kwargs):
        full = args + self.weights
        entry = self.op._pick(full, kwargs, pin=self.pin, accepted=self._accepted)
        return self.op._run(entry, full, kwargs, prepared=None if entry is None else self._prepared(entry))


def call_counts() -> dict[str, dict[str, int]]:
    return {name: dict(op.calls) for name, op in OPS.items() if op.calls}


def reset_call_counts() -> None:
    for op in OPS.values():
        op.calls.clear()
