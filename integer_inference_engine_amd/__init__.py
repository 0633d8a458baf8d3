"""imie — MI355X-native (gfx950) producer for the integer inference engine's hot path.

Packed Q1_0 and Q4_K/Q6_K integer dequant-matmul, fixed-point attention and the integer RMSNorm / RoPE / SiLU
kernels, as hand-written HIP behind a C-ABI (``libimie_gfx950.so``). ``gpu_native`` mirrors the Bonsai
producer interface; ``qk_gpu`` mirrors the north-mini-code one.
"""
from ._lib import LIB_PATH, device_available  # noqa: F401
