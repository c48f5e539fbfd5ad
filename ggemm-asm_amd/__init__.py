"""MI355X-native variable-K FP8 grouped weight-gradient GEMM.

``C[g] = s_lhs * s_rhs * LHS[offs[g]:offs[g+1]]^T @ RHS[offs[g]:offs[g+1]]`` with e4m3 x e5m2
inputs, fp32 accumulation and bf16 output, computed by hand-written gfx950 HIP kernels behind
the C ABI in include/ggemm_vark.h. Modules:

* ``vark``    -- torch ops over the C ABI (mirror of the reference's oracle op signature)
* ``harness`` -- code-object launch path mirroring the reference's hipModule harness
* ``inputs``  -- seeded generators for the measured configurations
* ``build``   -- in-tree hipcc build of the library and the drop-in code object
"""
from . import build, inputs  # noqa: F401
from ._lib import GGemmError, launch_geometry, library_path, load as load_library  # noqa: F401
from .vark import (as_bf16_bits, grouped_gemm_fp8_tensorwise_variable_k,  # noqa: F401
                   grouped_gemm_mxfp8_variable_k)

CODE_OBJECT_PATH = build.CO_PATH
