"""Op dispatch with FlashIM's plugin API (``flashim/ops/_registry.py:164-428``), for running this backend without
FlashIM installed. The same names and semantics:

* ``Op(name, reference, composite=, weights=)``; ``op.register(name, device=DeviceSpec(...), requires=, priority=,
  when=, prepare=, accepts=)(fn)`` adds an impl taking the reference's arguments;
* selection: available impls sorted by ``(-priority, device.span, registration order)``, negative priority = opt-in,
  then ``accepts(*weights)`` and ``when(*args, **kwargs)``;
* ``op.get(name)`` pins an impl (a pinned impl that does not apply runs the reference), ``op.bind(*weights)`` fixes
  the trailing weight operands and runs each impl's ``prepare`` once, ``op.explain``, ``op.supports``, call counts,
  ``FLASHIM_OPS`` overrides (``-op`` / ``op:impl``) and ``FLASHIM_STRICT_OPS``.

One deliberate difference: the op declarations of this package carry no torch implementation. Their "reference" is
:func:`no_reference`, which raises, because this package never computes a result outside its HIP kernels; the torch
references live in FlashIM (and, as the test oracle, in this repository's ``oracle/``). Registered into FlashIM
(:mod:`flashim_amd.plugin`), the impls sit next to FlashIM's real references, which then are the fallback.
"""

from __future__ import annotations

import os
from collections import Counter
from collections.abc import Callable, Iterable
from dataclasses import dataclass, field, fields, is_dataclass

import torch

from flashim_amd.platforms import Feature, Platform, platform_for

REFERENCE = "reference"


@dataclass(frozen=True)
class DeviceSpec:
    type: str
    min_capability: tuple[int, int] | None = None
    max_capability: tuple[int, int] | None = None

    def matches(self, platform: Platform) -> bool:
        if self.type not in ("*", platform.device_type):
            return False
        if self.min_capability is None and self.max_capability is None:
            return True
        if platform.capability is None:
            return False
        if self.min_capability is not None and platform.capability < self.min_capability:
            return False
        return self.max_capability is None or platform.capability <= self.max_capability

    @property
    def span(self) -> float:
        if self.type == "*":
            return float("inf")
        low = self.min_capability or (0, 0)
        high = self.max_capability or (99, 99)
        return (high[0] * 100 + high[1]) - (low[0] * 100 + low[1])


@dataclass
class Impl:
    name: str
    fn: Callable
    device: DeviceSpec
    requires: frozenset[Feature] = frozenset()
    priority: int = 0
    when: Callable[..., bool] | None = None
    order: int = 0
    weights: int = 0
    prepare: Callable[..., tuple] | None = None
    accepts: Callable[..., bool] | None = None

    @property
    def opt_in(self) -> bool:
        return self.priority < 0

    def available(self, platform: Platform) -> bool:
        return self.device.matches(platform) and platform.supports(*self.requires)

    def rejection(self, platform: Platform, args: tuple, kwargs: dict) -> str | None:
        if not self.device.matches(platform):
            return f"device {self.device} does not match {platform.device_type} {platform.arch}".rstrip()
        missing = sorted(f.value for f in self.requires if not platform.supports(f))
        if missing:
            return "missing features " + ",".join(missing)
        if self.accepts is not None and not self.accepts(*args[len(args) - self.weights:]):
            return "accepts() rejected the weights"
        if self.when is not None and not self.when(*args, **kwargs):
            return "when() rejected the arguments"
        return None


@dataclass
class _Config:
    disabled: set[str] = field(default_factory=set)
    forced: dict[str, str] = field(default_factory=dict)
    strict: bool = False


_CONFIG = _Config()
OPS: dict[str, Op] = {}


def configure(spec: str | None) -> None:
    """Apply a ``FLASHIM_OPS``-style override string (replacing earlier overrides)."""
    _CONFIG.disabled.clear()
    _CONFIG.forced.clear()
    for token in (spec or "").split(","):
        token = token.strip()
        if not token or token.startswith("+"):
            continue
        if token.startswith("-"):
            _CONFIG.disabled.add(token[1:])
        elif ":" in token:
            op, impl = token.split(":", 1)
            _CONFIG.forced[op] = impl
        else:
            raise ValueError(f"Invalid FLASHIM_OPS token {token!r}")


def set_strict(strict: bool) -> None:
    _CONFIG.strict = strict


configure(os.environ.get("FLASHIM_OPS"))
set_strict(os.environ.get("FLASHIM_STRICT_OPS", "0") == "1")


def no_reference(name: str) -> Callable:
    def reference(*args, **kwargs):
        raise NotImplementedError(
            f"op {name!r}: no HIP impl applies to these arguments and flashim_amd carries no torch fallback "
            "(register the backend into FlashIM for its reference path)"
        )

    reference.__name__ = f"_{name}_reference"
    return reference


def _first_device(values: Iterable) -> torch.device | None:
    for value in values:
        if isinstance(value, torch.Tensor):
            return value.device
        if is_dataclass(value) and not isinstance(value, type):
            value = [getattr(value, f.name) for f in fields(value)]
        if isinstance(value, (list, tuple)):
            device = _first_device(value)
            if device is not None:
                return device
    return None


class Op:
    def __init__(self, name: str, reference: Callable | None = None, *, composite: bool = False, weights: int = 0):
        if name in OPS:
            raise ValueError(f"Duplicate op {name!r}")
        self.name = name
        self.reference = reference if reference is not None else no_reference(name)
        self.composite = composite
        self.weights = weights
        self.impls: list[Impl] = []
        self.calls: Counter[str] = Counter()
        OPS[name] = self

    def register(self, name: str, *, device: DeviceSpec, requires: Iterable[Feature] = (), priority: int = 0,
                 when: Callable[..., bool] | None = None, prepare: Callable[..., tuple] | None = None,
                 accepts: Callable[..., bool] | None = None) -> Callable[[Callable], Callable]:
        if name == REFERENCE or any(impl.name == name for impl in self.impls):
            raise ValueError(f"Duplicate impl {name!r} for op {self.name!r}")
        if (prepare is not None or accepts is not None) and not self.weights:
            raise ValueError(f"Op {self.name!r} declares no weight operands to prepare or accept")

        def decorator(fn: Callable) -> Callable:
            self.impls.append(Impl(name, fn, device, frozenset(requires), priority, when, len(self.impls),
                                   self.weights, prepare, accepts))
            return fn

        return decorator

    def candidates(self, platform: Platform) -> list[Impl]:
        available = [impl for impl in self.impls if impl.available(platform)]
        return sorted(available, key=lambda i: (-i.priority, i.device.span, i.order))

    def _platform(self, args: tuple, kwargs: dict) -> Platform:
        return platform_for(_first_device(args) or _first_device(kwargs.values()) or torch.device("cpu"))

    def _find(self, name: str) -> Impl:
        for impl in self.impls:
            if impl.name == name:
                return impl
        raise ValueError(f"Op {self.name!r} has no impl {name!r} (registered: {[i.name for i in self.impls]})")

    def _choose(self, args: tuple, kwargs: dict, pin: str | None = None, accepted: dict[str, bool] | None = None,
                strict: bool = True) -> Impl | None:
        forced = _CONFIG.forced.get(self.name)
        if forced == REFERENCE or self.name in _CONFIG.disabled:
            return None
        if forced is not None:
            return self._find(forced)
        if pin == REFERENCE:
            return None
        platform = self._platform(args, kwargs)
        for impl in [self._find(pin)] if pin is not None else self.candidates(platform):
            if not impl.available(platform) or (pin is None and impl.opt_in):
                continue
            if impl.accepts is not None:
                ok = None if accepted is None else accepted.get(impl.name)
                if ok is None:
                    ok = bool(impl.accepts(*args[len(args) - impl.weights:]))
                    if accepted is not None:
                        accepted[impl.name] = ok
                if not ok:
                    continue
            if impl.when is None or impl.when(*args, **kwargs):
                return impl
        if pin is None and strict and _CONFIG.strict and platform.device_type != "cpu":
            raise RuntimeError(f"Op {self.name!r} fell back to the reference on {platform.describe()}")
        return None

    def explain(self, *args, **kwargs) -> dict[str, str]:
        platform = self._platform(args, kwargs)
        chosen, _ = self.select(*args, **kwargs)
        ranked = self.candidates(platform)
        ranked += [impl for impl in self.impls if impl not in ranked]
        report = {}
        for impl in ranked:
            if impl.name == chosen:
                report[impl.name] = "selected"
            else:
                reason = "opt-in (negative priority): pin it" if impl.opt_in else "lower priority"
                report[impl.name] = impl.rejection(platform, args, kwargs) or reason
        report[REFERENCE] = "selected" if chosen == REFERENCE else "fallback"
        return report

    def supports(self, *args, **kwargs) -> bool:
        return self._choose(args, kwargs, strict=False) is not None

    def select(self, *args, **kwargs) -> tuple[str, Callable]:
        impl = self._choose(args, kwargs)
        return (REFERENCE, self.reference) if impl is None else (impl.name, impl.fn)

    def _invoke(self, impl: Impl | None, args: tuple, kwargs: dict, prepared: tuple | None = None):
        if impl is None:
            self.calls[REFERENCE] += 1
            return self.reference(*args, **kwargs)
        call_args = args
        if impl.prepare is not None:
            split = len(args) - self.weights
            if prepared is None:
                prepared = tuple(impl.prepare(*args[split:]))
            call_args = args[:split] + prepared
        if not torch.compiler.is_compiling():
            self.calls[impl.name] += 1
        return impl.fn(*call_args, **kwargs)

    def __call__(self, *args, **kwargs):
        return self._invoke(self._choose(args, kwargs), args, kwargs)

    def get(self, name: str | None) -> Callable:
        if name is None:
            return self
        if name != REFERENCE:
            self._find(name)

        def pinned(*args, **kwargs):
            return self._invoke(self._choose(args, kwargs, pin=name), args, kwargs)

        return pinned

    def bind(self, *weights, impl: str | None = None) -> BoundOp:
        if len(weights) != self.weights:
            raise ValueError(f"Op {self.name!r} takes {self.weights} weight operands, got {len(weights)}")
        if impl is not None and impl != REFERENCE:
            self._find(impl)
        return BoundOp(self, weights, impl)

    def __repr__(self) -> str:
        return f"Op({self.name}: reference, {', '.join(i.name for i in self.impls)})"


class BoundOp:
    """An op with its trailing weight operands fixed; each impl's ``prepare`` runs once (``flashim/ops/_registry.py:366-424``)."""

    def __init__(self, op: Op, weights: tuple, pin: str | None = None) -> None:
        self.op, self.weights, self.pin = op, weights, pin
        self._prepared: dict[str, tuple] = {}
        self._accepted: dict[str, bool] = {}

    @property
    def platform(self) -> Platform:
        return platform_for(_first_device(self.weights) or torch.device("cpu"))

    def _usable(self) -> list[Impl]:
        impls = [i for i in self.op.candidates(self.platform) if i.accepts is None or i.accepts(*self.weights)]
        return impls if self.pin is None else [i for i in impls if i.name == self.pin]

    @property
    def available(self) -> list[str]:
        return [impl.name for impl in self._usable()]

    @property
    def primary(self) -> str:
        return next(iter(self.available), REFERENCE)

    def warmup(self) -> BoundOp:
        for impl in self._usable():
            if impl.prepare is not None and impl.name not in self._prepared:
                self._prepared[impl.name] = tuple(impl.prepare(*self.weights))
        return self

    def __call__(self, *args, **kwargs):
        full = args + self.weights
        impl = self.op._choose(full, kwargs, pin=self.pin, accepted=self._accepted)
        prepared = None
        if impl is not None and impl.prepare is not None:
            prepared = self._prepared.get(impl.name)
            if prepared is None:
                prepared = self._prepared[impl.name] = tuple(impl.prepare(*self.weights))
        return self.op._invoke(impl, full, kwargs, prepared=prepared)


def reset_call_counts() -> None:
    for op in OPS.values():
        op.calls.clear()


def call_counts() -> dict[str, dict[str, int]]:
    return {name: dict(op.calls) for name, op in OPS.items() if op.calls}
