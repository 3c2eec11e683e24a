"""Undeclared operator shapes the prepare-time variant modules are tested on (CPU: build and
load; GPU: parity of every variant). (input modes, output modes, cores' rank, dtype name)."""
JIT_SHAPES = [
    ((4, 6, 8), (6, 4, 8), 8, "float16"),        # a new shape at a compiled rank
    ((4, 6, 8), (6, 4, 8), 16, "float16"),
    ((4, 6, 8), (6, 4, 8), 12, "bfloat16"),      # rank 12: rank-16 kernels, zero-padded links
    ((16, 16, 20), (20, 16, 16), 8, "bfloat16"),  # the integration guide's example shape
    ((8, 12, 20), (12, 10, 24), 4, "float16"),   # rank 4 on the library's own rank-8 tables
    ((8, 12, 20), (12, 10, 24), 12, "float16"),  # rank 12 on the library's own rank-16 tables
    ((4, 6, 8), (6, 4, 8), 8, "float32"),        # fp32 on fp32 MFMAs
    ((8, 12, 20), (12, 10, 24), 16, "float32"),  # fp32 at rank 16 (a module: no fp32 R16 table)
]
