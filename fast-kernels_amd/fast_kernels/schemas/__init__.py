from fast_kernels.schemas.results import BenchmarkCase, ResultBundle, RunMetadata
from fast_kernels.schemas.suite import BenchmarkSuite, RegistryConfig, ShapeCase, ToleranceConfig

__all__ = [
    "BenchmarkCase",
    "BenchmarkSuite",
    "RegistryConfig",
    "ResultBundle",
    "RunMetadata",
    "ShapeCase",
    "ToleranceConfig",
]
