"""omniwave_amd — MI355X-native (gfx950) backend for the OmniWeave BiGEMM operator.

Public API mirrors the reference package (omniweave/__init__.py:5-8): ``create_model``,
``create_model_from_config`` and ``bigemm``; plus the route plans and the HIP entry points.
"""

__version__ = "0.1.0"

from omniwave_amd.bigemm import bigemm, register_backend
from omniwave_amd.block import enable_fp8
from omniwave_amd.hip import bigemm_block_hip, bigemm_delta_hip, hip_is_supported
from omniwave_amd.registry import create_model, create_model_from_config
from omniwave_amd.routing import RoutePlan, build_route_plan, build_stage_schedule

__all__ = [
    "RoutePlan",
    "bigemm",
    "bigemm_block_hip",
    "bigemm_delta_hip",
    "build_route_plan",
    "build_stage_schedule",
    "create_model",
    "create_model_from_config",
    "enable_fp8",
    "hip_is_supported",
    "register_backend",
]
