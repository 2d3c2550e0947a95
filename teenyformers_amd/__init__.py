"""teenyformers_amd: MI355X (gfx950) implementation of teenyformers' attention
hot path -- flash-attention 2 forward/backward, RoPE, head transposes, and the
Llama block's RMSNorm / SwiGLU / embedding kernels -- behind a C ABI
(include/teeny_hip.h, libteeny_hip.so).

Importing the package needs no GPU; the kernels load on first use and raise
if libteeny_hip.so has not been built (python -m teenyformers_amd.build).
"""

__all__ = ["ops"]
