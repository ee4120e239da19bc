"""dgen_hip: MI355X (gfx950) execution backend for DGen schedules.

The compute lives in libdgen_hip.so (HIP kernels + C ABI, include/dgen_hip.h);
this package is the host-side mirror of the reference's runtime interface
(LazyRuntime) plus the schedule builders for the benchmark workloads.
"""
from .program import Program  # noqa: F401
from .runtime import HIPError, HIPLazyRuntime, device_count, load_library  # noqa: F401
from .workloads import (BiquadConfig, HarmonicConfig, MembraneConfig, OscBankConfig, SplitMix64,  # noqa: F401
                        StftConfig, SvfConfig, SweptPhasorConfig)
