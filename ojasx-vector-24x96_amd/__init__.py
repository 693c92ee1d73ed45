"""MI355X-native split-manifold LUT execution path (OjasX drop-in).

Loaded under the module name ``ojasx_vector_24x96_amd`` (the directory name
is not an identifier; ``__graft_entry__.load_package()`` registers it).

Faces, each mirroring a reference interface:

* C-ABI ``libojasx_lut_hip.so`` (``include/ojasx_lut_c_api.h``): the reference
  C-ABI's 21 symbols plus device-pointer / stream variants
* ``native``: ``NativeSplitManifoldLinear``, ``NativeKVCache``,
  ``NativeSplitManifoldMoE``, ``get_engine_info`` (reference ctypes binding)
* ``engine``: ``SplitManifoldLUTLinear`` (reference PyTorch module)
* ``math_engine``: ``QuantizedWeight``, ``pack_codes``, ``unpack_codes``,
  ``subspace_lut_rvq_gemm`` (reference codec container and math engine)
* ``long_context``: ``PagedCompressedKVCache`` (reference int8 paged KV cache)
  and ``PagedCodeKVCache`` (paged codebook-code KV cache with device append
  and decode)
* ``decoder``: ``LUTDecoder`` / ``synthetic_decoder``, the 4B-shaped greedy
  decoder over LUT linears and the code KV cache (HIP graph per token)
* ``oqpack``: the reference's oqpack.v1 container (verify, mmap, write) and
  the loader of its residual-VQ linears as GPU LUT layers
* ``synthetic``: seeded synthetic inputs of the benchmark configurations
"""
from . import _lib
from ._lib import OjasxError, lib

__all__ = ["OjasxError", "lib", "native", "engine", "math_engine", "long_context", "decoder",
           "oqpack", "synthetic"]


def __getattr__(name):
    # Lazy submodules: ``engine`` imports torch, ``native`` only numpy.
    import importlib
    if name in ("native", "engine", "math_engine", "long_context", "decoder", "oqpack",
                "synthetic"):
        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(name)
