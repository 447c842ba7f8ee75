"""3dmaker_amd: MI355X-native (gfx950) per-sample training hot path of 3DMaker.

The product is the C-ABI shared library ``lib3dmaker_amd.so`` built from
``csrc/`` (declarations in ``include/*.h``).  This module binds it with ctypes
for Python callers, tests and the benchmark; it adds no compute of its own and
has no fallback: if the library is missing or a call fails, it raises.

Device buffers are passed as raw device pointers (ints) or as any object with
a ``data_ptr()`` method (e.g. torch tensors); streams as raw hipStream_t ints
(0 = null stream).
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib3dmaker_amd.so")

__all__ = [
    "LIB_PATH", "lib", "launch", "MLPOption", "MLPGridOptions", "HashGrid", "Net",
    "OUT_ACT_NONE", "OUT_ACT_SIGMOID", "ptr", "check", "Float3", "Uint3", "NerfOptions", "Nerf", "NerfTrainer", "NtrConfig", "NtrStats",
]

OUT_ACT_NONE = 0
OUT_ACT_SIGMOID = 1


class MLPOption(C.Structure):
    """modules/TinyMLP/TinyMLP.h:26-33"""
    _fields_ = [("inputDim", C.c_int), ("hiddenDim", C.c_int), ("outputDim", C.c_int),
                ("numLayers", C.c_int), ("activationType", C.c_int), ("outputActivation", C.c_int)]


class MLPGridOptions(C.Structure):
    """modules/TinyMLP/TinyMLPHashGrid.h:11-23"""
    _fields_ = [("vectorDim", C.c_int), ("hiddenDim", C.c_int), ("outputDim", C.c_int),
                ("numLayers", C.c_int), ("activationType", C.c_int), ("tableSize", C.c_int),
                ("numLevels", C.c_int), ("b", C.c_float), ("lowestSize", C.c_int),
                ("featuresLevel", C.c_int)]


class GridBuffers(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "master_hashtable", "fwd_hashtable", "hashtable_grads", "hash_m", "hash_v",
        "master_weights", "master_biases", "fwd_weights", "w_grad", "b_grad", "activations",
        "dx_out", "dloss", "padded_inputs", "padded_outputs")] + [("hw", MLPGridOptions), ("step", C.c_int)] + \
        [(n, C.c_void_p) for n in ("w_m", "w_v", "b_m", "b_v")]


class NetBuffers(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "master_weights", "master_biases", "fwd_weights", "w_grad", "b_grad", "activations",
        "dloss", "padded_outputs")] + [("hw", MLPOption), ("step", C.c_int)] + \
        [(n, C.c_void_p) for n in ("w_m", "w_v", "b_m", "b_v")]


class Float3(C.Structure):
    """HIP float3 passed by value (12 bytes)."""
    _fields_ = [("x", C.c_float), ("y", C.c_float), ("z", C.c_float)]


class Uint3(C.Structure):
    """HIP uint3 passed by value (12 bytes)."""
    _fields_ = [("x", C.c_uint), ("y", C.c_uint), ("z", C.c_uint)]


class NerfOptions(C.Structure):
    """modules/NeRF/InstantNerf.h:35-76 (byte layout of include/nerf_capi.h InerfOptions);
    start from Nerf.default_options()."""
    _fields_ = [("gridResolution", C.c_uint * 3), ("aabbMin", C.c_float * 3), ("aabbMax", C.c_float * 3),
                ("levelsMipmap", C.c_int), ("numCascades", C.c_int), ("samplesPerVoxel", C.c_int),
                ("densityHiddenDim", C.c_int), ("densityNumLayers", C.c_int),
                ("colorHiddenDim", C.c_int), ("colorNumLayers", C.c_int),
                ("hashTableSize", C.c_int), ("numLevels", C.c_int), ("growthFactor", C.c_float),
                ("baseResolution", C.c_int), ("featuresPerLevel", C.c_int),
                ("renderBatchSize", C.c_int), ("batchSize", C.c_int), ("rayChunkSize", C.c_int),
                ("lambdaDepth", C.c_float), ("lambdaDist", C.c_float), ("learningRate", C.c_float),
                ("beta1", C.c_float), ("beta2", C.c_float), ("epsilon", C.c_float), ("lossScale", C.c_float),
                ("bgColor", C.c_float * 3), ("minDensityThreshold", C.c_float), ("decayValue", C.c_float),
                ("densityBias", C.c_float), ("legacyRenderFlag", C.c_uint8), ("isProfiling", C.c_uint8)]


class NtrConfig(C.Structure):
    """modules/NeRF/NerfTrainer.h:27-41 (include/trainer_capi.h NtrConfig); start from NerfTrainer.default_config()."""
    _fields_ = [("lambdaDepth", C.c_float), ("lambdaDist", C.c_float), ("numCascades", C.c_int),
                ("minDensityThreshold", C.c_float), ("sampleK", C.c_int), ("batchSize", C.c_int),
                ("renderBatchSize", C.c_int), ("depthFraction", C.c_float), ("shouldValidate", C.c_uint8),
                ("maxLR", C.c_float), ("minLR", C.c_float), ("annealSteps", C.c_int)]


class NtrStats(C.Structure):
    """TrainStats (NerfTrainer.h:16-25)."""
    _fields_ = [("step", C.c_int), ("targetSteps", C.c_int), ("loss", C.c_float), ("psnr", C.c_float),
                ("lr", C.c_float), ("epochs", C.c_float), ("msPerStep", C.c_float), ("etaSeconds", C.c_float)]


class StepBuffers(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "num_steps", "ray_offsets", "positions", "ray_indices", "t_sorted", "density_out", "color_input",
        "color_output", "sigma", "render_rgb", "phi", "dw", "weight_sum", "dsigma", "color_dx", "density_grad",
        "result")] + [("trainSteps", C.c_int), ("windowStart", C.c_uint32), ("encodings", C.c_void_p),
                      ("encodingPlane", C.c_uint32), ("activationsSaved", C.c_int), ("density_stride", C.c_int)]


class RefreshBuffers(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("samples", "density_out", "tmp_grid", "active_list", "active_count")] + \
        [("last_count", C.c_int), ("density_stride", C.c_int), ("density_order", C.c_void_p)]


_vp, _i, _f, _u = C.c_void_p, C.c_int, C.c_float, C.c_uint
_u32 = C.c_uint32

# name -> (restype, argtypes); every symbol here is declared in include/*.h
SIGNATURES = {
    # include/tinymlp_abi.h (reference launchers)
    "launchNetworkFusionKernel": (None, [_vp, _vp, _vp, _vp, _vp, _i, _vp]),
    "launchNetworkFusionBackwardKernel": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp]),
    "launchNetworkFusionGradKernel": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp]),
    "launchAdamWeightsOptim": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _f, _f, _f, _f, _f, _f, _f, _vp]),
    "launchAdamBiasOptim": (None, [_vp, _vp, _vp, _vp, _vp, _f, _f, _f, _f, _f, _f, _f, _vp]),
    "launchMSELossGrad": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _f, _vp, _i]),
    "launchZeroGradients": (None, [_vp, _vp, _vp, _vp]),
    "launchNetworkFusionHashTableKernel": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp]),
    "launchNetworkFusionHashTableGradKernel": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp]),
    "launchNetworkFusionHashTableBackwardKernel": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp]),
    "launchNetworkFusionScatterBackwardKernel": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp]),
    "launchHashTableBackwardKernel": (None, [_vp, _vp, _vp, _i, _i, _i, _f, _i, _i, _vp]),
    "launchHashTableBackwardKernelNoAlloc": (None, [_vp, _vp, _vp, _i, _i, _i, _f, _i, _i, _vp]),
    "launchAdamHashGridOptim": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _f, _f, _f, _f, _f, _f, _f, _vp]),
    "launchHashEncodeKernel": (None, [_vp, _vp, _vp, _i, _vp, _i, _vp]),
    "tinymlp_last_error": (_i, []),
    "tinymlp_last_error_message": (C.c_char_p, []),
    # include/tinymlp_capi.h (flat handle API)
    "tmlp_grid_create": (_vp, [C.POINTER(MLPGridOptions), _i, _i, _u, _i]),
    "tmlp_grid_destroy": (None, [_vp]),
    "tmlp_grid_switch_mode": (_i, [_vp, _i]),
    "tmlp_grid_zero_grad": (_i, [_vp, _vp]),
    "tmlp_grid_forward": (_i, [_vp, _vp, _vp, _i, _vp]),
    "tmlp_grid_inference": (_i, [_vp, _vp, _vp, _i, _vp]),
    "tmlp_grid_loss": (_i, [_vp, _vp, _i, _f, _i, C.POINTER(_f), _vp]),
    "tmlp_grid_backward": (_i, [_vp, _vp, _i, _vp]),
    "tmlp_grid_set_split_scatter": (_i, [_vp, _i]),
    "tmlp_grid_step": (_i, [_vp, _f, _f, _f, _f, _f, _vp]),
    "tmlp_grid_scatter_adam_table": (_i, [_vp, _vp, _vp, _i, _i, _f, _f, _f, _f, _f, _vp, _vp]),
    "tmlp_grid_step_mlp": (_i, [_vp, _f, _f, _f, _f, _f, _vp]),
    "tmlp_grid_reset_step": (_i, [_vp]),
    "tmlp_grid_load_weights": (_i, [_vp, _vp, _vp]),
    "tmlp_grid_save_weights": (_i, [_vp, _vp, _vp]),
    "tmlp_grid_load_hashgrid": (_i, [_vp, _vp]),
    "tmlp_grid_save_hashgrid": (_i, [_vp, _vp]),
    "tmlp_grid_load_file": (_i, [_vp, C.c_char_p]),
    "tmlp_grid_save_file": (_i, [_vp, C.c_char_p]),
    "tmlp_grid_buffers": (_i, [_vp, C.POINTER(GridBuffers)]),
    "tmlp_net_create": (_vp, [C.POINTER(MLPOption), _i, _i, _u, _i]),
    "tmlp_net_destroy": (None, [_vp]),
    "tmlp_net_switch_mode": (_i, [_vp, _i]),
    "tmlp_net_zero_grad": (_i, [_vp, _vp]),
    "tmlp_net_forward": (_i, [_vp, _vp, _vp, _i, _vp]),
    "tmlp_net_inference": (_i, [_vp, _vp, _vp, _i, _vp]),
    "tmlp_net_loss": (_i, [_vp, _vp, _i, _f, _i, C.POINTER(_f), _vp]),
    "tmlp_net_backward": (_i, [_vp, _vp, _vp, _i, _vp]),
    "tmlp_net_step": (_i, [_vp, _f, _f, _f, _f, _f, _vp]),
    "tmlp_net_reset_step": (_i, [_vp]),
    "tmlp_net_load_weights": (_i, [_vp, _vp, _vp]),
    "tmlp_net_save_weights": (_i, [_vp, _vp, _vp]),
    "tmlp_net_load_file": (_i, [_vp, C.c_char_p]),
    "tmlp_net_save_file": (_i, [_vp, C.c_char_p]),
    "tmlp_net_buffers": (_i, [_vp, C.POINTER(NetBuffers)]),
    "tmlp_device_synchronize": (_i, []),
    # include/nerf_abi.h (NeRF launchers)
    "processRaysHitLinear": (_i, [_u32, _vp, _vp, _vp, _vp, _vp, _vp, Uint3, Float3, Float3, _i, _i, _i, _i,
                                  C.POINTER(_u32), _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "launchMarchRaysDDA": (None, [_u32, _vp, _vp, _vp, _vp, _vp, _vp, Uint3, Float3, Float3, _i, _i, _i, _vp, _vp,
                                  _vp, _vp]),
    "processRaysChunk": (None, [_u32, _vp, _vp, _vp, _vp, _vp, _vp, Uint3, Float3, Float3, _i, _i, _i, _vp, _vp, _vp,
                                _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "processRaysChunkLinear": (None, [_u32, _vp, _vp, _vp, _vp, _vp, _vp, Uint3, Float3, Float3, _i, _i, _i, _vp,
                                      _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "processRaysHitData": (None, [_u32, _vp, _vp, _vp, _vp, _vp, _vp, Uint3, Float3, Float3, _i, _i, _i, _vp, _vp,
                                  _vp, _vp]),
    "processRaysHitPositions": (_i, [_u32, _vp, _vp, _vp, _vp, _vp, _vp, Uint3, Float3, Float3, _i, _i, _i, _u32, _i,
                                     C.POINTER(_u32), C.POINTER(_u32), _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "launchComputeRealSHDegree3": (None, [_u32, _vp, _vp, _vp]),
    "launchVolumeRendering": (None, [_u32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _f,
                                     Float3, _u32, _u32, _vp]),
    "launchComputeRayAabbInv": (None, [_u32, _vp, _vp, Float3, Float3, _i, _vp, _vp, _vp, _vp]),
    "launchFetchRayChunk": (None, [_i, _i, _i, _u32, _i, _i, _i, _f, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _vp, _vp, _vp, _vp, _vp, _u32, _f, _f, _f, Float3, _i, _vp]),
    "launchComputeSHGather": (None, [_vp, _vp, _i, _i, _f, _vp, _vp, _vp, _vp]),
    "launchComputeColorGrad": (None, [_u32, _u32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _f,
                                      _u32, _vp]),
    "launchVolumeRenderingColorGrad": (None, [_u32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp,
                                              _vp, _f, _f, Float3, _vp, _vp, _i, _vp, _f, _f, _u32, _vp]),
    "launchComputeDensityGrad": (None, [_u32, _vp, _vp, _vp, _vp]),
    "launchUpdateMasterGrid": (None, [_vp, _vp, _f, _i, _vp]),
    "launchReduceSum": (None, [_vp, _i, _vp, _vp]),
    "launchUpdateOccupancyGrid": (None, [_vp, _vp, _vp, _i, _i, _i, _f, _f, _vp]),
    "launchBuildMipmaps": (None, [_vp, Uint3, _i, _i, _vp]),
    "nerfHeadsPackedBytes": (C.c_size_t, []),
    "launchNerfHeadsPack": (None, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "launchNerfHeadsForward": (None, [_vp, _vp, _i, _i, _vp, _vp, _i, _f, _i, _vp, _vp, _vp, _vp, _vp]),
    "launchNerfHeadsBackward": (None, [_vp, _vp, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp]),
    "launchNerfHeadsWeightGrads": (None, [_vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp]),
    "nerf_abi_echo_vec": (None, [Float3, Uint3, C.POINTER(_f)]),
    # include/nerf_capi.h (InstantNerf handle API)
    "inerf_default_options": (None, [C.POINTER(NerfOptions)]),
    "inerf_options_size": (C.c_size_t, []),
    "inerf_create": (_vp, [C.POINTER(NerfOptions)]),
    "inerf_destroy": (None, [_vp]),
    "inerf_train": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, C.POINTER(_i), _vp, _vp, _vp]),
    "inerf_set_learning_rate": (_i, [_vp, _f]),
    "inerf_set_next_rays": (_i, [_vp, _vp, _vp, _u32]),
    "inerf_set_bg_color": (_i, [_vp, _f, _f, _f]),
    "inerf_set_step_limit": (_i, [_vp, _i]),
    "inerf_set_keep_color_dx": (_i, [_vp, _i]),
    "inerf_last_rays_trained": (_u32, [_vp]),
    "inerf_set_profiling": (_i, [_vp, _i]),
    "inerf_print_stats": (_i, [_vp]),
    "inerf_stats": (_i, [_vp, C.c_char_p, _i]),
    "inerf_reset_stats": (_i, [_vp]),
    "inerf_set_memory_mode": (_i, [_vp, _i]),
    "inerf_render": (_i, [_vp, _vp, _vp, _u32, _vp, _vp]),
    "inerf_query_occupancy": (_i, [_vp, _vp, _i, _vp, _f, _vp]),
    "inerf_query_density_logit": (_i, [_vp, _vp, _i, _vp, _vp]),
    "inerf_query_radiance": (_i, [_vp, _vp, _i, _f, _f, _f, _vp, _vp]),
    "inerf_build_occupancy_bitgrid": (_i, [_vp, _vp, _f, _vp]),
    "inerf_update_occupancy": (_i, [_vp, _vp]),
    "inerf_occupancy_bytes": (C.c_size_t, [_vp]),
    "inerf_get_occupancy": (_i, [_vp, _vp]),
    "inerf_set_occupancy": (_i, [_vp, _vp]),
    "inerf_get_master_grid": (_i, [_vp, _vp]),
    "inerf_step_buffers": (_i, [_vp, C.POINTER(StepBuffers)]),
    "inerf_refresh_buffers": (_i, [_vp, C.POINTER(RefreshBuffers)]),
    "inerf_save": (_i, [_vp, C.c_char_p]),
    "inerf_load": (_i, [_vp, C.c_char_p]),
    "inerf_get_options": (_i, [_vp, C.POINTER(NerfOptions)]),
    "inerf_density": (_vp, [_vp]),
    "inerf_color": (_vp, [_vp]),
    "inerf_philox4x32_10": (None, [C.POINTER(_u32), _u32, _u32]),
    # include/trainer_capi.h
    "ntr_default_config": (None, [C.POINTER(NtrConfig)]),
    "ntr_create": (_vp, [C.POINTER(NtrConfig)]),
    "ntr_destroy": (None, [_vp]),
    "ntr_load_dataset": (_i, [_vp, _vp, _vp, _i, _i, _i, _f]),
    "ntr_begin_training": (_i, [_vp, _i]),
    "ntr_train_steps": (_i, [_vp, _i, C.POINTER(NtrStats)]),
    "ntr_validate": (_i, [_vp, C.POINTER(_f)]),
    "ntr_save": (_i, [_vp, C.c_char_p]),
    "ntr_load": (_i, [_vp, C.c_char_p]),
    "ntr_render_orbit": (_i, [_vp, _f, _f, _f, _f, _i, _i, _vp]),
    "ntr_render_train_view": (_i, [_vp, _i, _i, _i, _vp]),
    "ntr_num_train_views": (_i, [_vp]),
    "ntr_step": (_i, [_vp]),
    "ntr_num_cascades": (_i, [_vp]),
    "ntr_estimate_num_cascades": (_i, [_vp, _i]),
    "tmlp_version": (C.c_char_p, []),
}

_LIB = None


def lib():
    """Load lib3dmaker_amd.so (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def ptr(x) -> int | None:
    """Device pointer of x (int, None, or an object with data_ptr())."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return int(x.data_ptr())


def check(rc: int = None):
    """Raise RuntimeError if the last library call failed."""
    L = lib()
    if (rc is not None and rc != 0) or L.tinymlp_last_error() != 0:
        raise RuntimeError(L.tinymlp_last_error_message().decode())


def launch(name: str, *args):
    """Call a reference launcher from include/tinymlp_abi.h and raise on failure.

    Objects with data_ptr() are passed as their device pointer; ctypes
    structures should be passed by reference (ctypes.byref)."""
    L = lib()
    conv = [ptr(a) if hasattr(a, "data_ptr") else a for a in args]
    getattr(L, name)(*conv)
    check()


class HashGrid:
    """TinyMLPHashGrid (modules/TinyMLP/TinyMLPHashGrid.h:33-85) over the flat C API."""

    def __init__(self, opt: MLPGridOptions, max_batch: int, infer_batch: int = 0, seed: int = 42,
                 training: bool = True):
        self._L = lib()
        self.opt = opt
        self.h = self._L.tmlp_grid_create(C.byref(opt), max_batch, infer_batch, seed, int(training))
        if not self.h:
            check(1)

    def close(self):
        if getattr(self, "h", None):
            self._L.tmlp_grid_destroy(self.h)
            self.h = None

    __del__ = close

    def _c(self, rc):
        if rc != 0:
            check(rc)

    def switch_mode(self, training: bool):
        self._c(self._L.tmlp_grid_switch_mode(self.h, int(training)))

    def zero_grad(self, stream=0):
        self._c(self._L.tmlp_grid_zero_grad(self.h, stream))

    def forward(self, inputs, outputs, batch, stream=0):
        self._c(self._L.tmlp_grid_forward(self.h, ptr(inputs), ptr(outputs), batch, stream))

    def inference(self, inputs, outputs, batch, stream=0):
        self._c(self._L.tmlp_grid_inference(self.h, ptr(inputs), ptr(outputs), batch, stream))

    def calculate_loss_and_grad(self, targets, batch, loss_scale=65536.0, fetch_loss=False, stream=0):
        out = C.c_float(0.0)
        self._c(self._L.tmlp_grid_loss(self.h, ptr(targets), batch, loss_scale, int(fetch_loss),
                                       C.byref(out), stream))
        return out.value

    def backward(self, batch, custom_grad=None, stream=0):
        self._c(self._L.tmlp_grid_backward(self.h, ptr(custom_grad), batch, stream))

    def set_split_scatter(self, enabled: bool):
        self._c(self._L.tmlp_grid_set_split_scatter(self.h, int(enabled)))

    def step(self, lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, loss_scale=65536.0, stream=0):
        self._c(self._L.tmlp_grid_step(self.h, lr, beta1, beta2, eps, loss_scale, stream))

    def scatter_adam_table(self, dx, positions, n, pos_stride=4, lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8,
                           loss_scale=65536.0, stream=0, tile_live=None):
        """The table half of the next step, fused into the scatter of dx (TinyMLPHashGrid::scatterAdamTable);
        tile_live: optional uint32 per 16 rows of dx, 0 where the rows are all +-0 (skipped)."""
        self._c(self._L.tmlp_grid_scatter_adam_table(self.h, ptr(dx), ptr(positions), pos_stride, n, lr, beta1, beta2,
                                                     eps, loss_scale, ptr(tile_live), stream))

    def step_mlp(self, lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, loss_scale=65536.0, stream=0):
        self._c(self._L.tmlp_grid_step_mlp(self.h, lr, beta1, beta2, eps, loss_scale, stream))

    def reset_step(self):
        self._c(self._L.tmlp_grid_reset_step(self.h))

    def load_weights(self, w, b):
        self._c(self._L.tmlp_grid_load_weights(self.h, w.ctypes.data, b.ctypes.data))

    def save_weights(self, w, b):
        self._c(self._L.tmlp_grid_save_weights(self.h, w.ctypes.data, b.ctypes.data))

    def load_hashgrid(self, t):
        self._c(self._L.tmlp_grid_load_hashgrid(self.h, t.ctypes.data))

    def save_hashgrid(self, t):
        self._c(self._L.tmlp_grid_save_hashgrid(self.h, t.ctypes.data))

    def load_file(self, path: str):
        self._c(self._L.tmlp_grid_load_file(self.h, path.encode()))

    def save_file(self, path: str):
        self._c(self._L.tmlp_grid_save_file(self.h, path.encode()))

    def buffers(self) -> GridBuffers:
        b = GridBuffers()
        self._c(self._L.tmlp_grid_buffers(self.h, C.byref(b)))
        return b


class Net:
    """TinyMLP (modules/TinyMLP/TinyMLP.h:35-84) over the flat C API."""

    def __init__(self, opt: MLPOption, max_batch: int, infer_batch: int = 0, seed: int = 42,
                 training: bool = True):
        self._L = lib()
        self.opt = opt
        self.h = self._L.tmlp_net_create(C.byref(opt), max_batch, infer_batch, seed, int(training))
        if not self.h:
            check(1)

    def close(self):
        if getattr(self, "h", None):
            self._L.tmlp_net_destroy(self.h)
            self.h = None

    __del__ = close

    def _c(self, rc):
        if rc != 0:
            check(rc)

    def switch_mode(self, training: bool):
        self._c(self._L.tmlp_net_switch_mode(self.h, int(training)))

    def zero_grad(self, stream=0):
        self._c(self._L.tmlp_net_zero_grad(self.h, stream))

    def forward(self, inputs, outputs, batch, stream=0):
        self._c(self._L.tmlp_net_forward(self.h, ptr(inputs), ptr(outputs), batch, stream))

    def inference(self, inputs, outputs, batch, stream=0):
        self._c(self._L.tmlp_net_inference(self.h, ptr(inputs), ptr(outputs), batch, stream))

    def calculate_loss_and_grad(self, targets, batch, loss_scale=65536.0, fetch_loss=False, stream=0):
        out = C.c_float(0.0)
        self._c(self._L.tmlp_net_loss(self.h, ptr(targets), batch, loss_scale, int(fetch_loss),
                                      C.byref(out), stream))
        return out.value

    def backward(self, batch, custom_grad=None, dx_out=None, stream=0):
        self._c(self._L.tmlp_net_backward(self.h, ptr(custom_grad), ptr(dx_out), batch, stream))

    def step(self, lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, loss_scale=65536.0, stream=0):
        self._c(self._L.tmlp_net_step(self.h, lr, beta1, beta2, eps, loss_scale, stream))

    def reset_step(self):
        self._c(self._L.tmlp_net_reset_step(self.h))

    def load_weights(self, w, b):
        self._c(self._L.tmlp_net_load_weights(self.h, w.ctypes.data, b.ctypes.data))

    def save_weights(self, w, b):
        self._c(self._L.tmlp_net_save_weights(self.h, w.ctypes.data, b.ctypes.data))

    def load_file(self, path: str):
        self._c(self._L.tmlp_net_load_file(self.h, path.encode()))

    def save_file(self, path: str):
        self._c(self._L.tmlp_net_save_file(self.h, path.encode()))

    def buffers(self) -> NetBuffers:
        b = NetBuffers()
        self._c(self._L.tmlp_net_buffers(self.h, C.byref(b)))
        return b


def _grid_view(h, opt):
    v = HashGrid.__new__(HashGrid)
    v._L, v.opt, v.h = lib(), opt, h
    v.close = lambda: None
    return v


def _net_view(h, opt):
    v = Net.__new__(Net)
    v._L, v.opt, v.h = lib(), opt, h
    v.close = lambda: None
    return v


class Nerf:
    """InstantNerf (modules/NeRF/InstantNerf.h:279-335) over the flat C API (include/nerf_capi.h)."""

    @staticmethod
    def default_options() -> NerfOptions:
        o = NerfOptions()
        lib().inerf_default_options(C.byref(o))
        return o

    def __init__(self, opts: NerfOptions):
        self._L = lib()
        self.h = self._L.inerf_create(C.byref(opts))
        if not self.h:
            check(1)
        self._views(opts)

    def _views(self, opts: NerfOptions):
        self.opts = opts
        G = opts.gridResolution[0] * opts.gridResolution[1] * opts.gridResolution[2]
        self.cells = opts.numCascades * G
        dopt = MLPGridOptions(vectorDim=4, hiddenDim=opts.densityHiddenDim, outputDim=16,
                              numLayers=opts.densityNumLayers, activationType=0, tableSize=opts.hashTableSize,
                              numLevels=opts.numLevels, b=opts.growthFactor, lowestSize=opts.baseResolution,
                              featuresLevel=opts.featuresPerLevel)
        copt = MLPOption(inputDim=32, hiddenDim=opts.colorHiddenDim, outputDim=3, numLayers=opts.colorNumLayers,
                         activationType=0, outputActivation=OUT_ACT_SIGMOID)
        self.density = _grid_view(self._L.inerf_density(self.h), dopt)
        self.color = _net_view(self._L.inerf_color(self.h), copt)

    def close(self):
        if getattr(self, "h", None):
            self._L.inerf_destroy(self.h)
            self.h = None

    __del__ = close

    def _c(self, rc):
        if rc != 0:
            check(rc)

    def train(self, rays_o, rays_d, rgb_true, num_rays, rays_depth=None, rays_sigma=None, rgb_out=None, stream=0,
              max_steps=4096):
        """trainWithRaysHit; returns (steps taken, [compacted samples per step])."""
        cnt = C.c_int(0)
        # one step consumes >= 1 ray: room for num_rays counts; the buffer is
        # kept and grown, not allocated and zeroed on every call
        need = max(int(max_steps), int(num_rays), 1)
        if getattr(self, "_hits", None) is None or len(self._hits) < need:
            self._hits = (_u32 * need)()
        hits = self._hits
        self._c(self._L.inerf_train(self.h, ptr(rays_o), ptr(rays_d), ptr(rays_depth), ptr(rays_sigma),
                                    ptr(rgb_true), int(num_rays), C.byref(cnt), hits, ptr(rgb_out), stream))
        return cnt.value, hits[:cnt.value]

    def set_learning_rate(self, lr):
        self._c(self._L.inerf_set_learning_rate(self.h, float(lr)))

    def set_next_rays(self, rays_o, rays_d, num_rays):
        """setNextRays: the rays of the next train() call, already written; their first hit batch is
        compacted beside this call's last step."""
        self._c(self._L.inerf_set_next_rays(self.h, ptr(rays_o), ptr(rays_d), int(num_rays)))

    def set_step_limit(self, n):
        """At most n optimizer steps per train() call (0: no limit)."""
        self._c(self._L.inerf_set_step_limit(self.h, int(n)))

    def last_rays_trained(self):
        return int(self._L.inerf_last_rays_trained(self.h))

    def set_keep_color_dx(self, on):
        """Keep each step's colour dL/d(input) in step_buffers().color_dx (introspection; the step
        with recomputed activations does not store it otherwise)."""
        self._c(self._L.inerf_set_keep_color_dx(self.h, int(on)))

    def set_bg_color(self, r, g, b):
        self._c(self._L.inerf_set_bg_color(self.h, float(r), float(g), float(b)))

    def set_profiling(self, on):
        self._c(self._L.inerf_set_profiling(self.h, int(on)))

    def print_stats(self):
        self._c(self._L.inerf_print_stats(self.h))

    def stats(self) -> dict:
        """{stage: (mean ms, calls)} of the profiled steps (set_profiling(True))."""
        buf = C.create_string_buffer(8192)
        self._L.inerf_stats(self.h, buf, 8192)
        out = {}
        for ent in buf.value.decode().split(";"):
            if ent:
                name, ms, n = ent.split(":")
                out[name] = (float(ms), int(n))
        return out

    def reset_stats(self):
        self._c(self._L.inerf_reset_stats(self.h))

    def save(self, path: str):
        """.inerf file of the reference (InstantNerf.cu:1206-1276)."""
        self._c(self._L.inerf_save(self.h, os.fsencode(path)))

    def load(self, path: str):
        """Re-initialise from an .inerf file; the options become the file's."""
        self._c(self._L.inerf_load(self.h, os.fsencode(path)))
        o = NerfOptions()
        self._c(self._L.inerf_get_options(self.h, C.byref(o)))
        self._views(o)

    def set_memory_mode(self, inference: bool):
        """INFERENCE selects renderBatchSize as the render hit batch; training needs TRAINING."""
        self._c(self._L.inerf_set_memory_mode(self.h, int(bool(inference))))

    def render(self, rays_o, rays_d, num_rays, rgb_out, stream=0):
        """renderImageHit: rgb_out [num_rays x 3] (device)."""
        self._c(self._L.inerf_render(self.h, ptr(rays_o), ptr(rays_d), num_rays, ptr(rgb_out), stream))

    def query_occupancy(self, pos, n, words_out, min_optical, stream=0):
        self._c(self._L.inerf_query_occupancy(self.h, ptr(pos), n, ptr(words_out), min_optical, stream))

    def query_density_logit(self, pos, n, logit_out, stream=0):
        self._c(self._L.inerf_query_density_logit(self.h, ptr(pos), n, ptr(logit_out), stream))

    def query_radiance(self, pos, n, view_dir, rgb_out, stream=0):
        self._c(self._L.inerf_query_radiance(self.h, ptr(pos), n, float(view_dir[0]), float(view_dir[1]),
                                             float(view_dir[2]), ptr(rgb_out), stream))

    def build_occupancy_bitgrid(self, bits_out, min_density, stream=0):
        self._c(self._L.inerf_build_occupancy_bitgrid(self.h, ptr(bits_out), min_density, stream))

    def update_occupancy(self, stream=0):
        self._c(self._L.inerf_update_occupancy(self.h, stream))

    def occupancy(self):
        import numpy as np
        out = np.zeros(self._L.inerf_occupancy_bytes(self.h), np.uint8)
        self._c(self._L.inerf_get_occupancy(self.h, out.ctypes.data))
        return out

    def set_occupancy(self, bits):
        import numpy as np
        bits = np.ascontiguousarray(bits, np.uint8)
        assert bits.size == self._L.inerf_occupancy_bytes(self.h)
        self._c(self._L.inerf_set_occupancy(self.h, bits.ctypes.data))

    def master_grid(self):
        import numpy as np
        out = np.zeros(self.cells, np.float32)
        self._c(self._L.inerf_get_master_grid(self.h, out.ctypes.data))
        return out

    def step_buffers(self) -> StepBuffers:
        b = StepBuffers()
        self._c(self._L.inerf_step_buffers(self.h, C.byref(b)))
        return b

    def refresh_buffers(self) -> RefreshBuffers:
        b = RefreshBuffers()
        self._c(self._L.inerf_refresh_buffers(self.h, C.byref(b)))
        return b


class NerfTrainer:
    """INerfTrainer (modules/NeRF/NerfTrainer.h:43-112) over include/trainer_capi.h."""

    @staticmethod
    def default_config() -> NtrConfig:
        c = NtrConfig()
        lib().ntr_default_config(C.byref(c))
        return c

    def __init__(self, config: NtrConfig):
        self._L = lib()
        self.h = self._L.ntr_create(C.byref(config))
        if not self.h:
            check(1)

    def close(self):
        if self.h:
            self._L.ntr_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _c(self, rc):
        if rc:
            raise RuntimeError(self._L.tinymlp_last_error_message().decode())

    def load_dataset(self, rgba, transforms, focal):
        """rgba: uint8 [n, h, w, 4] (host); transforms: float32 [n, 16] row-major camera-to-world."""
        import numpy as np
        rgba = np.ascontiguousarray(rgba, np.uint8)
        tf = np.ascontiguousarray(transforms, np.float32)
        n, hh, ww = rgba.shape[:3]
        self._c(self._L.ntr_load_dataset(self.h, rgba.ctypes.data, tf.ctypes.data, n, ww, hh, float(focal)))

    def begin_training(self, total_steps):
        self._c(self._L.ntr_begin_training(self.h, int(total_steps)))

    def train_steps(self, n) -> NtrStats:
        st = NtrStats()
        self._c(self._L.ntr_train_steps(self.h, int(n), C.byref(st)))
        return st

    def validate(self) -> float:
        p = C.c_float(0)
        self._c(self._L.ntr_validate(self.h, C.byref(p)))
        return p.value

    def save(self, path):
        self._c(self._L.ntr_save(self.h, os.fsencode(path)))

    def load(self, path):
        self._c(self._L.ntr_load(self.h, os.fsencode(path)))

    def render_orbit(self, azimuth, elevation, radius, fov=50.0, width=800, height=800):
        import numpy as np
        out = np.zeros((height, width, 3), np.float32)
        self._c(self._L.ntr_render_orbit(self.h, float(azimuth), float(elevation), float(radius), float(fov), width,
                                         height, out.ctypes.data))
        return out

    def render_train_view(self, index, width, height):
        import numpy as np
        out = np.zeros((height, width, 3), np.float32)
        self._c(self._L.ntr_render_train_view(self.h, int(index), width, height, out.ctypes.data))
        return out

    def num_train_views(self) -> int:
        return self._L.ntr_num_train_views(self.h)

    def step(self) -> int:
        return self._L.ntr_step(self.h)

    def num_cascades(self) -> int:
        return self._L.ntr_num_cascades(self.h)


def estimate_num_cascades(transforms) -> int:
    """DataLoader::getNumCascades on float32 [n, 16] row-major camera-to-world matrices (host only)."""
    import numpy as np
    tf = np.ascontiguousarray(transforms, np.float32).reshape(-1, 16)
    return lib().ntr_estimate_num_cascades(tf.ctypes.data, tf.shape[0])
