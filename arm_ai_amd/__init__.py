"""arm_ai_amd: MI355X-native (gfx950) quantized-weight matmul for arm_ai's LlamaCandle path.

The product is libarm_ai_amd.so (HIP kernels behind the C ABI in include/aq.h);
this package holds its sources (csrc/), its build script and the Python mirror
of candle's QTensor / QMatMul used by tests and the benchmark.
"""
from .qmatmul import (  # noqa: F401
    Context,
    GgmlDType,
    QMatMul,
    QMatMulError,
    QTensor,
    act_bytes,
    device_count,
    quantize_act_device,
    quantize_q8_0,
    quantize_q8k,
)
from ._lib import AqError, LIB_PATH  # noqa: F401
