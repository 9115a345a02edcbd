"""MI355X-native routed-expert MoE path of ComfyUI-Drama3 (gfx950 HIP kernels behind the reference's Python API).

kernels.py and offload.py keep the reference's call surface (drama3/kernels.py, drama3/offload.py); moe.py is the
fused one-launch layer for A8 banks (formats.py).
"""
