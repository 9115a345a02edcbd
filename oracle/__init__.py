"""Oracle: CPU restatements of the routed-expert path's arithmetic, used only to check results.

Test infrastructure. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import anything from here,
and only to check results or to time the reference's CPU path; the product (comfyui-drama3_amd/drama3) never does.

  oracle/numerics.py  bf16 / e4m3 conversions, H256 rotation (closed forms)
  oracle/a8.py        the fused A8 layer (int8, W4, W6, FP8 banks): routing, quantizers, packing, exact dots, layer
  oracle/reference.py the reference's own kernels (drama3/kernels.py SOURCE) restated: route_experts, rotate_rows,
                      gemv_int8 / gemv_fp8 / gemv_codes, grouped_*, weighted_sum, and resident_decode / prefill
  oracle/cpu_path.py  the reference's CPU "dequant-then-matmul" path (drama3/offload.py:152-199), timed by bench.py
"""
