"""MI355X-native FP8 grouped GEMMs of an MoE layer.

The variable-K weight gradient ``C[g] = s_lhs * s_rhs * LHS[offs[g]:offs[g+1]]^T @
RHS[offs[g]:offs[g+1]]`` (e4m3 x e5m2) and the persistent forward / data-gradient GEMM
``out[r] = s_a * s_b * A[r] @ B[g]^T`` (e4m3 or e5m2 A, e4m3 B), fp32 accumulation, bf16 output,
computed by hand-written gfx950 HIP kernels behind the C ABI in include/ggemm_vark.h and
include/ggemm_persistent.h. Modules:

* ``vark``       -- variable-K wgrad torch ops over the C ABI (mirror of the reference's oracle op)
* ``persistent`` -- fwd/dgrad grouped GEMM torch op over the C ABI (same)
* ``quant``      -- FP8 quantization producer (per-tensor and MX with group padding) over the C ABI
* ``autograd``   -- the FP8 grouped linear layer (forward, dgrad, wgrad) as a torch autograd op
* ``harness``    -- code-object launch paths mirroring the reference's hipModule harness
* ``inputs``     -- seeded generators for the measured configurations
* ``build``      -- in-tree hipcc build of the library and the drop-in code objects
"""
from . import build, inputs  # noqa: F401
from ._lib import GGemmError, bf16_kernel, launch_geometry, library_path, load as load_library  # noqa: F401
from .autograd import FP8DelayedScaling, FP8WeightCache, GroupedLinearFP8, grouped_linear_fp8  # noqa: F401
from .persistent import grouped_gemm_fp8_tensorwise  # noqa: F401
from .quant import (amax, padded_rows, quantize_fp8_tensorwise, quantize_fp8_tensorwise_delayed,  # noqa: F401
                    quantize_fp8_tensorwise_transpose, quantize_fp8_tensorwise_transpose_delayed,
                    quantize_mxfp8_grouped)
from .vark import (as_bf16_bits, grouped_gemm_fp8_tensorwise_variable_k,  # noqa: F401
                   grouped_gemm_mxfp8_variable_k)

CODE_OBJECT_PATH = build.CO_PATH
PERSISTENT_CODE_OBJECT_PATHS = build.PERSISTENT_CO_PATHS
