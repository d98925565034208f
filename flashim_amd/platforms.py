"""Platform detection, mirroring FlashIM's ``flashim/platforms`` (``base.py:9-80``, ``detect.py:68-139``,
``others.py:16-30``): a device resolves to a :class:`Platform` whose ``device_type`` is the dispatch key impls register
for. ROCm devices (which torch calls ``"cuda"``) get the key ``"rocm"`` so NVIDIA-tuned kernels never select there.

This build adds the CDNA4 ISA features its kernels need (``Feature.HIP``, ``MFMA_I8``, ``MFMA_F8F6F4_SCALED``,
``FP8_E4M3``), detected from the device's ``gcnArchName``; FlashIM's own ROCm detector lists only ``CUDA_GRAPHS`` /
``TRITON``, so the plugin registration (:mod:`flashim_amd.plugin`) checks the architecture in its ``when`` predicates
instead.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum

import torch


class Vendor(str, Enum):
    NVIDIA = "nvidia"
    AMD = "amd"
    GENERIC = "generic"


class Feature(str, Enum):
    TRITON = "triton"
    CUDA_GRAPHS = "cuda_graphs"
    FP8_E4M3 = "fp8_e4m3"  # OCP E4M3 (float8_e4m3fn); gfx950 converts to it natively (gfx942 used the fnuz variant)
    HIP = "hip"  # the flashim_amd HIP library is built for this device's architecture
    MFMA_I8 = "mfma_i8"  # v_mfma_i32_16x16x64_i8 (gfx950)
    MFMA_F8F6F4_SCALED = "mfma_f8f6f4_scaled"  # v_mfma_scale_f32_16x16x128_f8f6f4: E8M0 block scales in the MFMA


# gfx950 (MI350X / MI355X): the architecture the library is built and validated for.
HIP_ARCHS = ("gfx950",)


@dataclass(frozen=True)
class Platform:
    device_type: str
    device_index: int | None = None
    name: str = ""
    capability: tuple[int, int] | None = None
    features: frozenset[Feature] = field(default_factory=frozenset)
    vendor: Vendor = Vendor.GENERIC
    arch: str = ""
    torch_device_type: str | None = None

    @property
    def device(self) -> torch.device:
        return torch.device(self.torch_device_type or self.device_type, self.device_index)

    def supports(self, *features: Feature) -> bool:
        return all(feature in self.features for feature in features)

    def describe(self) -> str:
        arch = f" {self.arch}" if self.arch else ""
        feats = ",".join(sorted(f.value for f in self.features)) or "-"
        return f"{self.device_type}{arch} ({self.name or 'unknown'}) features={feats}"


def rocm_features(arch: str) -> frozenset[Feature]:
    features = {Feature.CUDA_GRAPHS}
    if arch in HIP_ARCHS:
        features |= {Feature.HIP, Feature.MFMA_I8, Feature.MFMA_F8F6F4_SCALED, Feature.FP8_E4M3}
    return frozenset(features)


def detect_rocm(index: int) -> Platform:
    props = torch.cuda.get_device_properties(index)
    arch = getattr(props, "gcnArchName", "").split(":")[0]
    return Platform(
        device_type="rocm", device_index=index, name=torch.cuda.get_device_name(index), features=rocm_features(arch),
        vendor=Vendor.AMD, arch=arch, torch_device_type="cuda",
    )


_PLATFORMS: dict[tuple[str, int | None], Platform] = {}


def _detect(device: torch.device) -> Platform:
    if device.type == "cpu":
        return Platform(device_type="cpu", name="cpu")
    if device.type == "cuda":
        index = device.index if device.index is not None else torch.cuda.current_device()
        if torch.version.hip:
            return detect_rocm(index)
        major, minor = torch.cuda.get_device_capability(index)
        return Platform("cuda", index, torch.cuda.get_device_name(index), (major, minor), vendor=Vendor.NVIDIA,
                        arch=f"sm_{major}{minor}")
    return Platform(device_type=device.type, device_index=device.index, name=device.type)


def platform_for(device: torch.device | str | None = None) -> Platform:
    device = torch.device(device if device is not None else ("cuda" if torch.cuda.is_available() else "cpu"))
    key = (device.type, device.index)
    platform = _PLATFORMS.get(key)
    if platform is None:
        platform = _PLATFORMS[key] = _detect(device)
    return platform


@torch.compiler.assume_constant_result  # a process constant per device: keeps dispatch traceable under torch.compile
def _arch_is_gfx950(device_type: str, index: int | None) -> bool:
    return platform_for(torch.device(device_type, index)).arch in HIP_ARCHS


def is_gfx950(device: torch.device) -> bool:
    return device.type == "cuda" and _arch_is_gfx950(device.type, device.index)
