"""GGML tensor type codes used by the packed-linear surface.

The reference imports these from gguf-py (`gguf.GGMLQuantizationType`); gguf-py is not a dependency here, so the
codes the packed-linear path needs are restated with their ggml values. A source tensor is any object with
`.shape` (GGUF order, [k, n], a numpy array), `.tensor_type` and `.data` (the raw bytes), as in the reference's
tests (tests/python/test_fused_packed.py:41).
"""
import enum


class GGMLQuantizationType(enum.IntEnum):
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    I8 = 24
    I16 = 25
    I32 = 26
    I64 = 27
    F64 = 28
    BF16 = 30


# (values, bytes) per block of every type a GGUF container may hold that this package reads (ggml's type traits).
TYPE_SIZE = {
    GGMLQuantizationType.F32: (1, 4), GGMLQuantizationType.F16: (1, 2), GGMLQuantizationType.BF16: (1, 2),
    GGMLQuantizationType.F64: (1, 8), GGMLQuantizationType.I8: (1, 1), GGMLQuantizationType.I16: (1, 2),
    GGMLQuantizationType.I32: (1, 4), GGMLQuantizationType.I64: (1, 8),
    GGMLQuantizationType.Q4_0: (32, 18), GGMLQuantizationType.Q4_1: (32, 20), GGMLQuantizationType.Q5_0: (32, 22),
    GGMLQuantizationType.Q5_1: (32, 24), GGMLQuantizationType.Q8_0: (32, 34), GGMLQuantizationType.Q8_1: (32, 36),
    GGMLQuantizationType.Q2_K: (256, 84), GGMLQuantizationType.Q3_K: (256, 110), GGMLQuantizationType.Q4_K: (256, 144),
    GGMLQuantizationType.Q5_K: (256, 176), GGMLQuantizationType.Q6_K: (256, 210), GGMLQuantizationType.Q8_K: (256, 292),
}

# (block size in values, block size in bytes) of the block formats the packed layers accept.
BLOCK_LAYOUT = {
    GGMLQuantizationType.Q8_0: (32, 34),
    GGMLQuantizationType.Q4_0: (32, 18),
    GGMLQuantizationType.Q2_K: (256, 84),
    GGMLQuantizationType.Q4_K: (256, 144),
    GGMLQuantizationType.Q6_K: (256, 210),
}
