"""camelid_amd: MI355X (gfx950) resident decode/prefill backend for Camelid.

The compute path is hand-written HIP behind the C ABI in include/camelid_hip.h;
this package holds the ctypes host mirror of Camelid's CudaResidentDecode interface.
"""
from .engine import DeviceBuffer, EngineDims, HipResidentDecode, device_info  # noqa: F401
from .model import CONFIGS, ModelConfig, ResidentSession, SyntheticModel  # noqa: F401

__all__ = ["DeviceBuffer", "EngineDims", "HipResidentDecode", "device_info", "CONFIGS", "ModelConfig",
           "ResidentSession", "SyntheticModel"]
