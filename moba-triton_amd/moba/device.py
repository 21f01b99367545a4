"""Device facts for MI355X (gfx950) and result-row metadata.

Mirrors the reference's `src/moba/device.py` API (`TENSOR_CORE_TILE`,
`check_gathered_head_dim`, `supports_dtype`, `DeviceInfo`) with AMD facts:
an MFMA operand tile edge of 16, 64-wide wavefronts, 128-byte cache lines,
160 KiB of LDS per CU.
"""

from dataclasses import dataclass

import torch

# Architecture the HIP library is compiled for.
TARGET_ARCH = "gfx950"

# Smallest block a KV tile may have: the MFMA operand edge (16x16x32 /
# 32x32x16 bf16 tiles are built from 16-wide K slices).
TENSOR_CORE_TILE = 16

# A gathered query row costs one cache line when it fills one.
CACHE_LINE_BYTES = 128

WAVEFRONT_SIZE = 64
LDS_BYTES_PER_CU = 160 * 1024


def check_gathered_head_dim(head_dim: int, itemsize: int) -> tuple[bool, str]:
    """head_dim must be a power of two whose row fills a cache line
    (`device.py:96-120`)."""
    if head_dim <= 0 or head_dim & (head_dim - 1):
        return False, f"head_dim {head_dim} must be a power of two"
    row_bytes = head_dim * itemsize
    if row_bytes < CACHE_LINE_BYTES:
        return False, (
            f"head_dim {head_dim} gives a {row_bytes}-byte row, below the "
            f"{CACHE_LINE_BYTES}-byte cache line; gathered rows would waste "
            "the remainder of every line fetched")
    return True, ""


def supports_dtype(dtype: torch.dtype, arch: str = TARGET_ARCH) -> tuple[bool, str]:
    """Whether the library computes in `dtype` on `arch` (`device.py:123-148`)."""
    if not str(arch).startswith(TARGET_ARCH):
        return False, f"library is built for {TARGET_ARCH}, found {arch}"
    if dtype not in (torch.bfloat16, torch.float16, torch.float32):
        return False, f"unsupported dtype {dtype}"
    return True, ""


def device_arch(index: int = 0) -> str:
    """gcnArchName of a visible device, e.g. 'gfx950:sramecc+:xnack-'."""
    props = torch.cuda.get_device_properties(index)
    return getattr(props, "gcnArchName", "") or ""


@dataclass(frozen=True)
class DeviceInfo:
    """Identifying metadata of the GPU a result was measured on
    (`device.py:150-207`)."""

    name: str
    arch: str
    total_memory_mb: int
    compute_units: int
    torch_version: str
    hip_version: str

    @classmethod
    def probe(cls, index: int = 0) -> "DeviceInfo":
        if not torch.cuda.is_available():
            raise RuntimeError("No GPU device available")
        p = torch.cuda.get_device_properties(index)
        return cls(
            name=p.name,
            arch=getattr(p, "gcnArchName", ""),
            total_memory_mb=p.total_memory // (1024 * 1024),
            compute_units=p.multi_processor_count,
            torch_version=torch.__version__,
            hip_version=str(torch.version.hip),
        )

    def as_row(self) -> dict:
        return {
            "gpu_name": self.name,
            "arch": self.arch,
            "total_memory_mb": self.total_memory_mb,
            "compute_units": self.compute_units,
            "torch_version": self.torch_version,
            "hip_version": self.hip_version,
        }
