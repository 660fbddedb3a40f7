"""torch dtype aliases used by the aiter API (aiter/utility/dtypes.py)."""
import torch

fp4x2 = getattr(torch, "float4_e2m1fn_x2", torch.uint8)
fp8_e8m0 = getattr(torch, "float8_e8m0fnu", torch.uint8)
fp8 = torch.float8_e4m3fn  # gfx950 uses the OCP e4m3fn encoding
bf16 = torch.bfloat16
fp16 = torch.float16
fp32 = torch.float32
u8 = torch.uint8
i32 = torch.int32
