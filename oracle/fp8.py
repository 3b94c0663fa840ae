"""FP8 e4m3 KV quantization, restated (test oracle only).

reference: vllm_rlt/core/kv_cache_manager.py:37-65 (``FP8_E4M3_MAX = 448``,
``quantize_fp8`` with a reciprocal-multiply scale clamped at fp32 ``tiny``,
saturating clamp before the OCP ``float8_e4m3fn`` cast, ``dequantize_fp8``).
"""

import torch

FP8_E4M3_MAX = 448.0


def quantize_fp8(x, fixed_scale=None):
    x = x.float()
    if fixed_scale is None:
        scale = (x.abs().amax(-1) * (1.0 / FP8_E4M3_MAX)).clamp_min(torch.finfo(torch.float32).tiny)
    else:
        scale = torch.full(x.shape[:-1], fixed_scale, dtype=torch.float32, device=x.device)
    codes = (x / scale.unsqueeze(-1)).clamp(-FP8_E4M3_MAX, FP8_E4M3_MAX)
    return codes.to(torch.float8_e4m3fn), scale


def dequantize_fp8(codes, scale, dtype):
    return (codes.float() * scale.unsqueeze(-1)).to(dtype)
