"""The C-ABI library loads and exports every function declared in include/*.h (no GPU)."""
import ctypes
import os
import re

import pytest

from helpers import pkg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")

C_HEADERS = [f for f in sorted(os.listdir(INCLUDE)) if f.endswith(".h")]


def declared_c_functions(path):
    """Names of functions declared inside extern "C" / plain-C headers."""
    src = open(path).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    if "class " in src:   # C++ class headers: only their extern "C" blocks count
        blocks = re.findall(r'extern "C"\s*\{(.*?)\n\}', src, flags=re.S)
        src = "\n".join(blocks)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b([A-Za-z_]\w*)\s*\([^;{]*\)\s*;", src, flags=re.M)
    return sorted(set(n for n in names if n not in ("if", "while", "for", "return")))


def test_headers_exist():
    assert "tinymlp_abi.h" in C_HEADERS and "tinymlp_capi.h" in C_HEADERS


@pytest.mark.parametrize("header", [h for h in C_HEADERS])
def test_library_exports_every_declared_symbol(header):
    L = ctypes.CDLL(pkg().LIB_PATH)
    names = declared_c_functions(os.path.join(INCLUDE, header))
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"{header}: not exported: {missing}"


def test_reference_launchers_present():
    names = declared_c_functions(os.path.join(INCLUDE, "tinymlp_abi.h"))
    for n in ["launchNetworkFusionKernel", "launchNetworkFusionBackwardKernel", "launchNetworkFusionGradKernel",
              "launchAdamWeightsOptim", "launchAdamBiasOptim", "launchMSELossGrad", "launchZeroGradients",
              "launchNetworkFusionHashTableKernel", "launchNetworkFusionHashTableGradKernel",
              "launchNetworkFusionHashTableBackwardKernel", "launchNetworkFusionScatterBackwardKernel",
              "launchHashTableBackwardKernel", "launchAdamHashGridOptim"]:
        assert n in names
    # the extern "C" launchers of modules/NeRF/InstantNerf.h:385-568
    names = declared_c_functions(os.path.join(INCLUDE, "nerf_abi.h"))
    for n in ["launchMarchRaysDDA", "processRaysChunk", "processRaysChunkLinear", "processRaysHitLinear",
              "launchComputeRealSHDegree3", "launchVolumeRendering", "processRaysHitData", "processRaysHitPositions"]:
        assert n in names


def test_launcher_argument_errors_without_gpu():
    """Argument errors of the march / SH launchers are reported before any device call."""
    P = pkg()
    L = P.lib()
    L.launchComputeRealSHDegree3(4, 16, 20, None)     # output not 16-byte aligned
    assert L.tinymlp_last_error() != 0 and b"aligned" in L.tinymlp_last_error_message()
    L.launchComputeRealSHDegree3(0, None, None, None)  # nothing to do
    assert L.tinymlp_last_error() == 0
    args = [None] * 6 + [P.Uint3(16, 16, 16), P.Float3(-1, -1, -1), P.Float3(1, 1, 1), 1, 1, 1]
    L.processRaysHitPositions(8, *args, 0, 64, None, None, None, None, None, None, None, None, None, None)
    assert L.tinymlp_last_error() != 0 and b"NULL" in L.tinymlp_last_error_message()
    L.processRaysChunk(8, *args, None, None, None, None, None, None, None, None, None, None, None, None)
    assert L.tinymlp_last_error() != 0 and b"NULL" in L.tinymlp_last_error_message()
    assert L.nerfHeadsPackedBytes() > 0
    fake = 1 << 20  # never dereferenced: every check below fails before a device call
    L.launchNerfHeadsForward(fake, fake, 64, 16, fake, fake, -1, 0.0, 1, fake, None, fake, fake, None)
    assert L.tinymlp_last_error() != 0 and b"num_samples" in L.tinymlp_last_error_message()
    L.launchNerfHeadsForward(fake, fake, 16, 16, fake, fake, 64, 0.0, 1, fake, None, fake, fake, None)
    assert L.tinymlp_last_error() != 0 and b"plane" in L.tinymlp_last_error_message()
    L.launchNerfHeadsForward(fake, fake, 64, 17, fake, fake, 64, 0.0, 1, fake, None, fake, fake, None)
    assert L.tinymlp_last_error() != 0 and b"levels" in L.tinymlp_last_error_message()
    L.launchNerfHeadsBackward(fake, fake, 64, 16, None, fake, fake, 64, fake, None, None, None, None)
    assert L.tinymlp_last_error() != 0 and b"null" in L.tinymlp_last_error_message()
    L.launchNerfHeadsWeightGrads(fake, fake, 64, 16, fake, fake, fake, None, None, 64, None, fake, fake, fake, None)
    assert L.tinymlp_last_error() != 0 and b"null" in L.tinymlp_last_error_message()
    L.launchNerfHeadsPack(None, fake, fake, fake, fake, None)
    assert L.tinymlp_last_error() != 0 and b"null" in L.tinymlp_last_error_message()


def test_python_bindings_cover_the_headers():
    names = set()
    for h in C_HEADERS:
        names.update(declared_c_functions(os.path.join(INCLUDE, h)))
    bound = set(pkg().SIGNATURES)
    assert names <= bound, f"declared but not bound: {sorted(names - bound)}"


def test_error_reporting_without_gpu():
    """An invalid shape is reported, not silently ignored (no device work is launched)."""
    P = pkg()
    opt = P.MLPOption(inputDim=32, hiddenDim=256, outputDim=16, numLayers=2, activationType=0, outputActivation=0)
    P.lib().launchNetworkFusionKernel(ctypes.byref(opt), None, None, None, None, 16, None)
    assert P.lib().tinymlp_last_error() != 0
    assert b"128" in P.lib().tinymlp_last_error_message()
