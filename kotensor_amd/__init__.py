"""kotensor_amd: MI355X (gfx950) implementation of Kotensor's group-wise INT8/INT4
weight-only quantization path.

The product is ``libkotensor_hip.so`` (C ABI: ``include/kotensor_hip.h``). This
package is a host-side mirror of the reference's API over that ABI:
``Quantization``, ``QuantizedTensor``, ``MatMul.multiply_quantized``,
``DeviceTensor.matmul_dequant(_into)``, ``QuantizedLinear``, the saveQuantized
file format (``SafeTensorsFile``, ``save_quantized``, ``load_quantized``) and the
device-resident decoder around the projections (``Transformer``, ``KVCache``,
``InferenceBuffers``, ``RoPEScaling``) and the fused projection + cross-entropy with a
quantized head (``fused_cross_entropy_loss``).
"""
from ._lib import IllegalArgumentException, IllegalStateException, LibraryMissingError, LIBRARY_PATH
from .device import DeviceBuffer, Stream, synchronize, device_count
from .quantization import Quantization, QuantizedTensor
from .matmul import MatMul, DeviceTensor
from .linear import QuantizedLinear, projection, forward_into_group
from .safetensors import SafeTensorsFile, save_entries, save_quantized, load_quantized
from .transformer import Transformer, KVCache, InferenceBuffers, RoPEScaling
from .loss import fused_cross_entropy_loss, FusedLoss, IGNORE_INDEX

__all__ = [
    "IllegalArgumentException",
    "IllegalStateException",
    "LibraryMissingError",
    "LIBRARY_PATH",
    "DeviceBuffer",
    "Stream",
    "synchronize",
    "device_count",
    "Quantization",
    "QuantizedTensor",
    "MatMul",
    "DeviceTensor",
    "QuantizedLinear",
    "projection",
    "forward_into_group",
    "SafeTensorsFile",
    "save_entries",
    "save_quantized",
    "load_quantized",
    "Transformer",
    "KVCache",
    "InferenceBuffers",
    "RoPEScaling",
    "fused_cross_entropy_loss",
    "FusedLoss",
    "IGNORE_INDEX",
]
