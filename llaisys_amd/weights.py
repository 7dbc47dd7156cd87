"""Device-resident weight upload: the op-side half of the reference loader's _map_weight.

The reference loader (python/llaisys/models/qwen2.py:114-147) upcasts every bf16 / f16
weight to a float32 numpy array and loads it into an F32 CPU tensor.  Here a weight goes to
HBM in the format the ops read:

* ``upload(array, DataType.BF16)`` -- one host-to-device copy when the host array already
  holds bf16 bits (a bf16 safetensors tensor read without upcasting:
  ``t.view(torch.int16).numpy().view(np.uint16)``); a float32 / float16 host array is
  copied as it is and converted on the device by llaisysCast, with the reference's rules
  (src/utils/types.hpp:116-139), so the result equals the reference's cast of each value.
* ``upload_int8(array)`` -- the weight in its host format, then llaisysQuantizeInt8 per
  output row on the device: INT8 codes [out, in] plus F32 scales [out], the format of
  llaisysLinearW8A16; the full-precision device copy is freed.

Host formats (llaisys_amd.hostfmt): numpy float32, float16, or uint16 holding bf16 bits.
"""
import numpy as np

from .libllaisys import DataType, DeviceType
from .ops import Ops
from .tensor import Tensor

_HOST_DTYPE = {np.dtype(np.float32): DataType.F32, np.dtype(np.float16): DataType.F16,
               np.dtype(np.uint16): DataType.BF16}


def _host_dtype(array):
    try:
        return _HOST_DTYPE[np.asarray(array).dtype]
    except KeyError:
        raise TypeError("weights are float32, float16 or uint16 (bf16 bits) arrays") from None


def _staged(array, device_id):
    """The host array on the device in its own format (one tensorLoad)."""
    a = np.ascontiguousarray(array)
    return Tensor.from_numpy(a, _host_dtype(a), device=DeviceType.AMD, device_id=device_id)


def upload(array, dtype: DataType = DataType.BF16, device_id: int = 0) -> Tensor:
    """Host weight -> AMD tensor of `dtype` (F32 / BF16 / F16), converted on the device."""
    if dtype not in (DataType.F32, DataType.BF16, DataType.F16):
        raise ValueError("upload: dtype must be F32, BF16 or F16 (use upload_int8 for INT8)")
    staged = _staged(array, device_id)
    if staged.dtype() == dtype:
        return staged
    out = Tensor(staged.shape(), dtype, device=DeviceType.AMD, device_id=device_id)
    Ops.cast(out, staged)
    return out


def upload_int8(array, device_id: int = 0):
    """Host weight [out, in] -> (codes I8 [out, in], scales F32 [out]) on the device, by
    llaisysQuantizeInt8 of the weight in its host format."""
    a = np.asarray(array)
    if a.ndim != 2:
        raise ValueError("upload_int8: weight must be 2-D [out_features, in_features]")
    staged = _staged(a, device_id)
    codes = Tensor(a.shape, DataType.I8, device=DeviceType.AMD, device_id=device_id)
    scales = Tensor((a.shape[0],), DataType.F32, device=DeviceType.AMD, device_id=device_id)
    Ops.quantize_int8(codes, scales, staged)
    return codes, scales
