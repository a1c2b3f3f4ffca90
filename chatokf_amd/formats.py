"""GGUF block formats on the path: ggml type ids and sizes.

Type ids follow ``LLM/Base/GGUF.swift:3-14``; bytes per row follow
``GGUF.rowByteCount`` (``LLM/Base/GGUF.swift:160-188``) and elements per block
follow ``GQ.blockElems`` (``LLM/Gemma/Gemma4Quant.swift:77-87``).
"""
Q4_0 = 2
Q8_0 = 8
IQ4_NL = 20
Q4_K = 12
Q5_K = 13
Q6_K = 14
IQ4_XS = 23
IQ2_XS = 17
IQ3_XXS = 18
IQ1_S = 19
IQ3_S = 21
IQ2_S = 22
IQ1_M = 29
F32 = 0
F16 = 1
BF16 = 30
Q2_K = 10
Q3_K = 11
IQ2_XXS = 16
Q2_0 = 42

NAMES = {Q8_0: "q8_0", Q4_K: "q4_k", IQ2_XXS: "iq2_xxs", Q2_0: "q2_0", Q4_0: "q4_0", IQ4_NL: "iq4_nl",
         Q5_K: "q5_k", Q6_K: "q6_k", IQ4_XS: "iq4_xs", IQ2_XS: "iq2_xs", IQ2_S: "iq2_s",
         IQ3_XXS: "iq3_xxs", IQ3_S: "iq3_s", IQ1_S: "iq1_s", IQ1_M: "iq1_m", F32: "f32", F16: "f16",
         BF16: "bf16", Q2_K: "q2_k", Q3_K: "q3_k"}
BY_NAME = {v: k for k, v in NAMES.items()}

# type -> (weights per block, bytes per block)
BLOCK = {Q8_0: (32, 34), Q2_0: (128, 34), Q4_K: (256, 144), IQ2_XXS: (256, 66), Q4_0: (32, 18),
         IQ4_NL: (32, 18), Q5_K: (256, 176), Q6_K: (256, 210), IQ4_XS: (256, 136),
         IQ2_XS: (256, 74), IQ2_S: (256, 82), IQ3_XXS: (256, 98), IQ3_S: (256, 110), IQ1_S: (256, 50),
         IQ1_M: (256, 56), Q2_K: (256, 84), Q3_K: (256, 110), F32: (32, 128), F16: (32, 64), BF16: (32, 64)}


def block_elems(t: int) -> int:
    return BLOCK[t][0]


def row_bytes(t: int, n: int) -> int:
    """Bytes of one row of n weights; n must be a whole number of blocks
    (any n for the plain f32 / f16 / bf16 types)."""
    if t in (F32, F16, BF16):
        return n * (4 if t == F32 else 2)
    e, b = BLOCK[t]
    if n % e:
        raise ValueError(f"{NAMES[t]} rows need a multiple of {e} weights, got {n}")
    return n // e * b
