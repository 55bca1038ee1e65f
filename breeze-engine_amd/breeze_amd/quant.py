"""MatMulNBits weight decode (the packing/dequant contract).

Same function, layout and semantics as breeze/quant.py:9-58, so ``A @ W``
with the dense result matches the quantized matmul up to activation
quantization.
"""
import numpy as np


def _unpack_nibbles(x, count):
    out = np.empty(x.shape[:-1] + (count,), np.uint8)
    out[..., 0::2] = x & 0x0F
    out[..., 1::2] = x >> 4
    return out


def dequantize_matmul_nbits(qweight, scales, qzeros, *, bits, block_size, K, N):
    """Dense fp32 ``W [K, N]`` with ``w = (q - zero_point) * scale`` per block.

    4-bit: qweight uint8 [N, n_blocks, block_size/2], low nibble first;
           qzeros packed 4-bit [N * ceil(n_blocks/2)] or None (zero point 8).
    8-bit: qweight uint8 [N, n_blocks, block_size]; qzeros [N, n_blocks] or
           None (zero point 128).
    scales: [N * n_blocks] (any float dtype)."""
    if bits not in (4, 8):
        raise NotImplementedError(f"MatMulNBits bits={bits} not supported (only 4, 8).")
    nb = (K + block_size - 1) // block_size
    sc = np.asarray(scales, dtype=np.float32).reshape(N, nb)
    have_zp = qzeros is not None and np.size(qzeros) > 0
    if bits == 8:
        q = np.ascontiguousarray(qweight).reshape(N, nb, block_size).astype(np.float32)
        zp = (np.ascontiguousarray(qzeros).reshape(N, nb).astype(np.float32) if have_zp
              else np.full((N, nb), 128.0, np.float32))
    else:
        packed = np.ascontiguousarray(qweight).reshape(N, nb, block_size // 2)
        q = _unpack_nibbles(packed, block_size).astype(np.float32)
        if have_zp:
            cols = (nb + 1) // 2
            zp = _unpack_nibbles(np.ascontiguousarray(qzeros).reshape(N, cols), 2 * cols)
            zp = zp[:, :nb].astype(np.float32)
        else:
            zp = np.full((N, nb), 8.0, np.float32)
    w = (q - zp[:, :, None]) * sc[:, :, None]
    return np.ascontiguousarray(w.reshape(N, nb * block_size)[:, :K].T)
