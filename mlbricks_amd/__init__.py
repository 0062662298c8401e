"""MI355X-native ElasticBit quantized linear, drop-in for the ElasticBit path of MLBricks.

    import mlbricks_amd as mlb
    model = mlb.ElasticBit.compress(model, calibrationData=batches, threshold=0.01)

The compute path is the HIP library ``mlbricks_amd/lib/libelasticbit_hip.so``
(build with ``python -m mlbricks_amd.csrc.build``); its C ABI is
``include/elasticbit.h``.
"""
from .elasticbit import BackendInfo, BitAnalysis, BitCandidate, ElasticBit, RuntimeMatrix
from .planner import AUTO_OPERATOR_DEFAULTS, EXECUTION_PLANNER, MLBricksExecutionPlanner
from .runtime import backend_report, normalize_backend, set_module_backend

__version__ = "0.1.0"

__all__ = [
    "ElasticBit",
    "RuntimeMatrix",
    "BitAnalysis",
    "BitCandidate",
    "BackendInfo",
    "AUTO_OPERATOR_DEFAULTS",
    "EXECUTION_PLANNER",
    "MLBricksExecutionPlanner",
    "normalize_backend",
    "set_module_backend",
    "backend_report",
]
