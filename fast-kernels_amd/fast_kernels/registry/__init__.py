from fast_kernels.registry.baselines import BaselineSpec, baseline_registry
from fast_kernels.registry.kernels import KernelSpec, kernel_registry

__all__ = ["BaselineSpec", "KernelSpec", "baseline_registry", "kernel_registry"]
