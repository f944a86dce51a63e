"""MI355X (gfx950) quantized-matmul ops with the Python surface of the reference's src/lfm2opt package.

kernels.ext() / kernels.int8_ext() return the op namespaces; int8.Int8Linear and quant.* mirror the reference's
INT8 linear layer and weight formats. All compute runs in liblfm2q.so (HIP, gfx950).
"""
