"""The benchmark configurations: projection shapes of each workload.

A projection is (name, quant type, N, K): W is [N][K], y = W . x.
"""
from .ops import Q4_K, Q6_K, Q8_0

# Config 1: single Q4_K GEMV (FFN gate/up of Qwen2.5-3B), seed 0.
SINGLE_Q4K = [("gate", Q4_K, 11008, 2048)]


def decode_layer(hidden, q_heads, kv_heads, head_dim, ffn):
    """Q4_K_M decode layer: Q, K, V, O, gate, up in Q4_K; down in Q6_K."""
    return [
        ("q", Q4_K, q_heads * head_dim, hidden),
        ("k", Q4_K, kv_heads * head_dim, hidden),
        ("v", Q4_K, kv_heads * head_dim, hidden),
        ("o", Q4_K, hidden, q_heads * head_dim),
        ("gate", Q4_K, ffn, hidden),
        ("up", Q4_K, ffn, hidden),
        ("down", Q6_K, hidden, ffn),
    ]


# The launches of a decode layer, as the reference's forward pass issues
# them (runtime/backends/cuda/native/transformer_forward.cu:474-980): one
# grouped Q8_1 GEMV for Q/K/V (GemvQ8_1Triple, :542) over the quantized
# attention-norm output, O accumulated into the fp32 residual
# (GemvQ8_1AccumF32, :726), one grouped launch for gate/up (GemvQ8_1Pair,
# :559) and down accumulated into the residual (:817).
# (launch name, projections, activation input, accumulate into Y)
DECODE_LAUNCHES = [
    ("qkv", ("q", "k", "v"), "attn_in", False),
    ("o", ("o",), "attn_out", True),
    ("gate_up", ("gate", "up"), "ffn_in", False),
    ("down", ("down",), "ffn_act", True),
]


# Config 2: Qwen2.5-3B layer (hidden 2048, 16/2 heads x 128, FFN 11008), M = 1, 4, 8.
QWEN3B_LAYER = decode_layer(2048, 16, 2, 128, 11008)
QWEN3B_LAYERS = 36
# Config 3: LM head at vocab 151936 x 2048, Q8_0 and Q6_K, M = 1, 8.
LM_HEAD = {"q8_0": [("lm_head", Q8_0, 151936, 2048)], "q6_k": [("lm_head", Q6_K, 151936, 2048)]}
# Config 4: Qwen2.5-14B layer (hidden 5120, 40/8 heads x 128, FFN 13824), M = 16, 32.
QWEN14B_LAYER = decode_layer(5120, 40, 8, 128, 13824)
QWEN14B_LAYERS = 48
# Config 5: Qwen2.5-32B prefill GEMMs (hidden 5120, FFN 27648), M = 512.
PREFILL_32B = [("ffn_up", Q4_K, 27648, 5120), ("ffn_down", Q6_K, 5120, 27648)]
