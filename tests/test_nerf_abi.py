"""Host-side checks of the NeRF C-ABI (no GPU): by-value vector arguments, the
NerfOptions mirror, and the occupancy sampler's Philox4x32-10 against the
known-answer vectors of Random123 (Salmon et al., SC'11, kat_vectors)."""
import ctypes as C

import pytest

from helpers import pkg


def test_float3_uint3_by_value():
    P = pkg()
    out = (C.c_float * 6)()
    P.lib().nerf_abi_echo_vec(P.Float3(1.5, -2.25, 3.125), P.Uint3(7, 8, 4000000000), out)
    assert list(out) == [1.5, -2.25, 3.125, 7.0, 8.0, 4000000000.0]


def test_nerf_options_mirror_and_defaults():
    P = pkg()
    assert P.lib().inerf_options_size() == C.sizeof(P.NerfOptions)
    o = P.Nerf.default_options()
    # InstantNerf.h:35-76 defaults
    assert list(o.gridResolution) == [128, 128, 128]
    assert list(o.aabbMin) == [-1.0] * 3 and list(o.aabbMax) == [1.0] * 3
    assert (o.levelsMipmap, o.numCascades, o.samplesPerVoxel) == (4, 1, 1)
    assert (o.densityHiddenDim, o.densityNumLayers, o.colorHiddenDim, o.colorNumLayers) == (64, 2, 64, 2)
    assert (o.hashTableSize, o.numLevels, o.baseResolution, o.featuresPerLevel) == (1 << 19, 16, 16, 2)
    assert abs(o.growthFactor - 1.3819) < 1e-6
    assert (o.renderBatchSize, o.batchSize, o.rayChunkSize) == (2048 * 1024, 256 * 1024, 256 * 1024)
    assert abs(o.lambdaDepth - 0.02882) < 1e-7 and abs(o.lambdaDist - 0.0362781) < 1e-7
    assert abs(o.learningRate - 1e-3) < 1e-9 and abs(o.beta2 - 0.999) < 1e-7 and o.lossScale == 1.0
    assert list(o.bgColor) == [1.0] * 3 and abs(o.minDensityThreshold - 0.01) < 1e-9
    assert abs(o.decayValue - 0.95) < 1e-7 and o.densityBias == 1.0
    assert o.legacyRenderFlag == 0 and o.isProfiling == 0


@pytest.mark.parametrize("ctr,key,want", [
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff, 0xffffffff), (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
])
def test_philox4x32_10_known_answers(ctr, key, want):
    c = (C.c_uint32 * 4)(*ctr)
    pkg().lib().inerf_philox4x32_10(c, key[0], key[1])
    assert tuple(c) == want


def test_inference_compositing_zero_rays_is_a_no_op():
    """d_dw_out NULL selects the inference compositor; zero rays launch nothing."""
    P = pkg()
    P.lib().launchVolumeRendering(0, None, None, None, None, None, None, None, None, None, None, None, None, None,
                                  0.0, 0.0, P.Float3(1, 1, 1), 0, 0, None)
    assert P.lib().tinymlp_last_error() == 0
