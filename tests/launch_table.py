"""Every launch the benchmark times, at its production shape, with the
kernel instance the dispatch must route it to.

tests/test_dispatch.py checks the routing on the CPU (dry-run launch log, no
GPU); tests/test_gpu_launches.py runs each launch on the GPU, asserts the
same kernel instance ran and checks the output against the oracle on
sampled rows.  A change of a dispatch threshold therefore fails on the CPU
until the table names the new kernel, and the GPU suite then covers it.

Entry kinds:
  gemv                ifx_qgemv, store
  *_ws                the same through ifx_qgemv_ws / ifx_qgemv_grouped_ws (K splits
                      reduced in split order through a workspace)
  gemv_accum          ifx_qgemv, accumulate into an fp32 residual
  grouped             ifx_qgemv_grouped (Q/K/V triple, gate/up pair), store
  grouped_rmsnorm     ifx_qgemv_grouped_rmsnorm (RMSNorm + Q8_1 fused in), store
  quantize_accum      ifx_qgemv_grouped_rmsnorm with norm_weight NULL (Q8_1 fused in), accumulate
  gate_up_silu_rmsnorm  ifx_qgemv_gate_up_silu_rmsnorm (Q8_1 output of silu(gate)*up)
  gate_up_silu        ifx_qgemv_gate_up_silu (Q8_1 output of silu(gate)*up)
  mmq_accum           ifx_qgemv_mmq on the down-projection MMQ layout (ifx_mmq_layout_build of
                      the raw type named), accumulate into an fp32 residual; _ws: ordered
                      K splits through the layout's own workspace
  prefill             ifx_qgemm_prefill
  prefill_int8        ifx_qgemm_prefill_kernel(IFX_PREFILL_INT8)
Kernel names: include/ifx_qgemm.h, ifx_launch_log_begin.
"""
Q8_0, Q4_K, Q6_K = 8, 12, 14
Q8_0_R, Q6_K_R = 108, 114  # row-split copies (ifx_repack) of Q8_0 / Q6_K rows
Q8_0_T, Q4_K_T, Q6_K_T = 208, 212, 214  # tiled copies (ifx_repack_tiled)

# 3B: hidden 2048, Q/K/V 2048/256/256, FFN 11008; 14B: hidden 5120, Q/K/V
# 5120/1024/1024, FFN 13824 (inferflux_amd/workloads.py)
QKV3, QKV14 = (2048, 256, 256), (5120, 1024, 1024)

# (id, entry, quant type, M, Ns, K, expected kernel instances)
LAUNCHES = [
    # config 1: single Q4_K GEMV 11008 x 2048
    ("c1_m1", "gemv", Q4_K, 1, (11008,), 2048, ["k_gemv<12,1,2,1,4,0,2>"]),
    ("c1_m8", "gemv", Q4_K, 8, (11008,), 2048, ["k_gemv_slot<12,8,8,0,0>"]),
    # config 2: the 3B decode layer as the reference launches it
    ("c2_qkv_m1", "grouped", Q4_K, 1, QKV3, 2048, ["k_gemv<12,1,1,1,4,0,2>"]),
    ("c2_o_m1", "gemv_accum", Q4_K, 1, (2048,), 2048, ["k_gemv<12,1,1,1,4,0,2,0,1>"]),
    ("c2_gate_up_m1", "grouped", Q4_K, 1, (11008, 11008), 2048, ["k_gemv<12,1,2,1,4,0,2>"]),
    ("c2_down_m1", "gemv_accum", Q6_K, 1, (2048,), 11008, ["k_gemv<14,1,2,3,1,0,1,0,1>"]),
    ("c2_down_r_m1", "gemv_accum", Q6_K_R, 1, (2048,), 11008, ["k_gemv<114,1,2,3,1,0,1,0,1>"]),
    ("c2_qkv_m4", "grouped", Q4_K, 4, QKV3, 2048, ["k_gemv_slot<12,8,8,0,0>"]),
    ("c2_o_m4", "gemv_accum", Q4_K, 4, (2048,), 2048, ["k_gemv_slot<12,8,8,0,3>"]),
    ("c2_gate_up_m4", "grouped", Q4_K, 4, (11008, 11008), 2048, ["k_gemv_lds<4,2,2,8,0>"]),
    ("c2_down_m4", "gemv_accum", Q6_K, 4, (2048,), 11008, ["k_gemv_slot<14,8,4,0,1>"]),
    ("c2_qkv_m8", "grouped", Q4_K, 8, QKV3, 2048, ["k_gemv_slot<12,8,8,0,0>"]),
    ("c2_o_m8", "gemv_accum", Q4_K, 8, (2048,), 2048, ["k_gemv_slot<12,8,8,0,3>"]),
    ("c2_gate_up_m8", "grouped", Q4_K, 8, (11008, 11008), 2048, ["k_gemv_slot<12,8,8,0,0>"]),
    ("c2_down_m8", "gemv_accum", Q6_K, 8, (2048,), 11008, ["k_gemv_slot<14,8,4,0,1>"]),
    # config 2 at M = 4 / 8 with SiLU * up + Q8_1 in the gate/up epilogue
    ("c2s_gate_up_m4", "gate_up_silu", Q4_K, 4, (11008,), 2048, ["k_gemv_slot<12,8,4,0,0,1>"]),
    ("c2s_gate_up_m8", "gate_up_silu", Q4_K, 8, (11008,), 2048, ["k_gemv_slot<12,8,4,0,0,1>"]),
    # config 2, the fused layer form the benchmark's step uses at M = 1
    ("c2f_qkv_m1", "grouped_rmsnorm", Q4_K, 1, QKV3, 2048, ["k_gemv<12,1,2,1,4,0,2,1>"]),
    ("c2f_o_m1", "quantize_accum", Q4_K, 1, (2048,), 2048, ["k_gemv<12,1,1,1,4,0,2,3,1>"]),
    ("c2f_gate_up_m1", "gate_up_silu_rmsnorm", Q4_K, 1, (11008,), 2048,
     ["k_gemv_swiglu_wide<1,0,1,8>"]),
    # config 3: LM head 151936 x 2048
    ("c3_q8_0_m1", "gemv", Q8_0, 1, (151936,), 2048, ["k_gemv<8,1,4,1,4,0,1>"]),
    ("c3_q8_0_m8", "gemv", Q8_0, 8, (151936,), 2048, ["k_mmvq<8,1,1,0>"]),
    ("c3_q6_k_m1", "gemv", Q6_K, 1, (151936,), 2048, ["k_gemv<14,1,4,1,4,0,2>"]),
    ("c3_q6_k_m8", "gemv", Q6_K, 8, (151936,), 2048, ["k_gemv_slot<14,8,1,0,0>"]),
    ("c3_q8_0_r_m1", "gemv", Q8_0_R, 1, (151936,), 2048, ["k_gemv<108,1,1,1,4,0,1>"]),
    ("c3_q6_k_r_m1", "gemv", Q6_K_R, 1, (151936,), 2048, ["k_gemv<114,1,4,1,4,0,2>"]),
    # config 4: the 14B decode layer at M = 16 / 32, and its Q4_K launches at M = 1 / 8
    ("c4_qkv_m16", "grouped", Q4_K, 16, QKV14, 5120, ["k_mmvq<12,1,8,0>"]),
    ("c4_o_m16", "gemv_accum", Q4_K, 16, (5120,), 5120, ["k_gemv_dq<12,0,1>"]),
    ("c4_gate_up_m16", "grouped", Q4_K, 16, (13824, 13824), 5120, ["k_mmvq<12,1,2,0>"]),
    ("c4_down_m1", "gemv_accum", Q6_K, 1, (5120,), 13824, ["k_gemv<14,1,4,4,1,0,1,0,1>"]),
    ("c4_down_m16", "gemv_accum", Q6_K, 16, (5120,), 13824, ["k_gemv_dq<14,0,1>"]),
    ("c4_qkv_m32", "grouped", Q4_K, 32, QKV14, 5120, ["k_fill_zero", "k_gemv_dq<12,0,1>"]),
    ("c4_o_m32", "gemv_accum", Q4_K, 32, (5120,), 5120, ["k_gemv_dq<12,0,1>"]),
    ("c4_gate_up_m32", "grouped", Q4_K, 32, (13824, 13824), 5120, ["k_gemv_dqr<12,0,0,0,4,2,8>"]),
    ("c4_down_m32", "gemv_accum", Q6_K, 32, (5120,), 13824, ["k_gemv_dq<14,0,1>"]),
    ("c4_qkv_m1", "grouped", Q4_K, 1, QKV14, 5120, ["k_gemv<12,1,1,1,4,0,4>"]),
    ("c4_o_m1", "gemv_accum", Q4_K, 1, (5120,), 5120, ["k_gemv<12,1,1,1,4,0,4,0,1>"]),
    ("c4_gate_up_m1", "grouped", Q4_K, 1, (13824, 13824), 5120, ["k_gemv<12,1,2,1,4,0,4>"]),
    ("c4_qkv_m8", "grouped", Q4_K, 8, QKV14, 5120, ["k_gemv_slot<12,8,8,0,0>"]),
    ("c4_o_m8", "gemv_accum", Q4_K, 8, (5120,), 5120, ["k_gemv_slot<12,8,8,0,3>"]),
    ("c4_gate_up_m8", "grouped", Q4_K, 8, (13824, 13824), 5120, ["k_gemv_slot<12,8,8,0,0>"]),
    # the benchmark's tiled forms: config 1 at M = 8, the 3B layer at M = 4 / 8
    # and the 14B layer at M = 16 / 32 with ordered K splits, the LM head at M = 8
    ("c1_m8_tiled", "gemv", Q4_K_T, 8, (11008,), 2048, ["k_gemv_slot<12,8,8,0,0,0,1>"]),
    ("c2t_qkv_m4", "grouped_ws", Q4_K_T, 4, QKV3, 2048, ["k_gemv_slot<12,8,8,0,0,0,1>"]),
    ("c2t_o_m4", "gemv_accum_ws", Q4_K_T, 4, (2048,), 2048, ["k_gemv_slot<12,8,8,0,3,0,1>"]),
    ("c2t_gate_up_m4", "gate_up_silu", Q4_K_T, 4, (11008,), 2048,
     ["k_gemv_slot<12,8,4,0,0,1,1>"]),
    ("c2t_down_m4", "gemv_accum_ws", Q6_K_T, 4, (2048,), 11008, ["k_gemv_slot<14,8,4,0,2,0,1>"]),
    ("c2t_qkv_m8", "grouped_ws", Q4_K_T, 8, QKV3, 2048, ["k_gemv_slot<12,8,8,0,0,0,1>"]),
    ("c2t_o_m8", "gemv_accum_ws", Q4_K_T, 8, (2048,), 2048, ["k_gemv_slot<12,8,8,0,3,0,1>"]),
    ("c2t_gate_up_m8", "gate_up_silu", Q4_K_T, 8, (11008,), 2048,
     ["k_gemv_slot<12,8,4,0,0,1,1>"]),
    ("c2t_down_m8", "gemv_accum_ws", Q6_K_T, 8, (2048,), 11008, ["k_gemv_slot<14,8,4,0,2,0,1>"]),
    ("c3_q8_0_t_m8", "gemv", Q8_0_T, 8, (151936,), 2048, ["k_gemv_slot<8,8,1,0,0,0,1>"]),
    ("c3_q6_k_t_m8", "gemv", Q6_K_T, 8, (151936,), 2048, ["k_gemv_slot<14,8,1,0,0,0,1>"]),
    ("c4t_qkv_m16", "grouped_ws", Q4_K_T, 16, QKV14, 5120, ["k_gemv_slot<12,16,8,0,0,0,1>"]),
    ("c4t_o_m16", "gemv_accum_ws", Q4_K_T, 16, (5120,), 5120, ["k_gemv_slot<12,16,8,0,3,0,1>"]),
    ("c4t_gate_up_m16", "grouped_ws", Q4_K_T, 16, (13824, 13824), 5120,
     ["k_gemv_dqr<12,0,1,0,8,4,8>"]),
    ("c4t_down_m16", "gemv_accum_ws", Q6_K_T, 16, (5120,), 13824,
     ["k_gemv_slot<14,16,4,0,2,0,1>"]),
    # plain accumulate launches at 9 <= M <= 16: the fp16-dequant GEMV's atomic split
    ("c4tp_o_m16", "gemv_accum", Q4_K_T, 16, (5120,), 5120, ["k_gemv_dq<12,0,1,1>"]),
    ("c4tp_down_m16", "gemv_accum", Q6_K_T, 16, (5120,), 13824, ["k_gemv_dq<14,0,1,1>"]),
    ("c2tp_o_m12", "gemv_accum", Q4_K_T, 12, (2048,), 2048, ["k_gemv_dq<12,0,1,1>"]),
    ("c4t_gate_up_silu_m16", "gate_up_silu", Q4_K_T, 16, (13824,), 5120,
     ["k_gemv_dqr<12,0,1,1,8,4,8>"]),
    ("c4t_gate_up_silu_m32", "gate_up_silu", Q4_K_T, 32, (13824,), 5120,
     ["k_gemv_dqr<12,0,1,1,4,2,8>"]),
    ("c4t_qkv_m32", "grouped_ws", Q4_K_T, 32, QKV14, 5120, ["k_gemv_dq<12,0,2,1>"]),
    ("c4t_o_m32", "gemv_accum_ws", Q4_K_T, 32, (5120,), 5120, ["k_gemv_dq<12,0,2,1>"]),
    ("c4t_gate_up_m32", "grouped_ws", Q4_K_T, 32, (13824, 13824), 5120,
     ["k_gemv_dqr<12,0,1,0,4,2,8>"]),
    ("c4t_down_m32", "gemv_accum_ws", Q6_K_T, 32, (5120,), 13824, ["k_gemv_dq<14,0,2,1>"]),
    # the down projections on the MMQ layout (FusedQuantGemm::DownProjMmq):
    # row-split rows at M <= 2, tiles above, ordered K splits
    ("c2m_down_m1", "mmq_accum", Q6_K, 1, (2048,), 11008, ["k_gemv<114,1,2,3,1,0,1,0,1>"]),
    ("c2m_down_m4", "mmq_accum_ws", Q6_K, 4, (2048,), 11008, ["k_gemv_slot<14,8,4,0,2,0,1>"]),
    ("c2m_down_m8", "mmq_accum_ws", Q6_K, 8, (2048,), 11008, ["k_gemv_slot<14,8,4,0,2,0,1>"]),
    ("c4m_down_m16", "mmq_accum_ws", Q6_K, 16, (5120,), 13824,
     ["k_gemv_slot<14,16,4,0,2,0,1>"]),
    ("c4m_down_m32", "mmq_accum_ws", Q6_K, 32, (5120,), 13824, ["k_gemv_dq<14,0,2,1>"]),
    # packed (per-row symmetric int8) activations at M = 1: config 1, the 3B
    # QKV triple and down projection, the 14B gate/up pair
    ("c1_packed_m1", "packed", Q4_K, 1, (11008,), 2048, ["k_gemv_packed<12,1,2>"]),
    ("c2_qkv_packed_m1", "packed", Q4_K, 1, QKV3, 2048, ["k_gemv_packed<12,1,2>"]),
    ("c2_down_packed_m1", "packed", Q6_K, 1, (2048,), 11008, ["k_gemv_packed<14,1,1>"]),
    ("c4_gate_up_packed_m1", "packed", Q4_K, 1, (13824, 13824), 5120, ["k_gemv_packed<12,1,4>"]),
    # config 5: 32B prefill GEMMs at M = 512 (default dispatch, and the int8 kernel)
    ("c5_up", "prefill", Q4_K, 512, (27648,), 5120, ["k_gemm_f16<12,8,0,0,0>"]),
    ("c5_down", "prefill", Q6_K, 512, (5120,), 27648, ["k_fill_zero", "k_gemm_f16<14,8,0,1,0>"]),
    ("c5_up_int8", "prefill_int8", Q4_K, 512, (27648,), 5120, ["k_gemm_mfma<12,2,0>"]),
    ("c5_down_int8", "prefill_int8", Q6_K, 512, (5120,), 27648, ["k_gemm_mfma<14,1,0>"]),
]

IDS = [l[0] for l in LAUNCHES]
