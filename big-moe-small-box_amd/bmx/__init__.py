"""bmx: MI355X-native routed-expert MoE layer (HIP kernels for gfx950 behind a C ABI, PyTorch-ROCm host)."""
from . import _lib
from ._lib import (ACT_GELU, ACT_RELU2, ACT_SILU, ACT_SILU_OAI, LANE_ADMIT, LANE_CPU, LANE_HOME, LANE_VRAM, PATH_AUTO,
                   PATH_DECODE, PATH_MID, PATH_PREFILL, PATH_SPLIT, SCORE_SIGMOID, SCORE_SOFTMAX, SCORE_SQRTSP, TF_K2, TF_K3, TF_K4,
                   TF_K25, TILE_BYTES, BmxError, lib)
from .experts import ExpertTable
from .layer import MoELayer
from .slots import ExpertSlots
from . import ops
from . import store
from . import cpu_lane
from .store import ExpertStore

__all__ = ["ExpertTable", "ExpertSlots", "ExpertStore", "MoELayer", "ops", "store", "cpu_lane", "lib", "BmxError", "TF_K2", "TF_K25", "TF_K3", "TF_K4", "TILE_BYTES",
           "SCORE_SIGMOID", "SCORE_SOFTMAX", "SCORE_SQRTSP", "ACT_SILU", "ACT_GELU", "ACT_RELU2", "ACT_SILU_OAI", "PATH_AUTO",
           "PATH_DECODE", "PATH_MID", "PATH_PREFILL", "PATH_SPLIT", "LANE_VRAM", "LANE_ADMIT", "LANE_HOME", "LANE_CPU", "_lib"]
