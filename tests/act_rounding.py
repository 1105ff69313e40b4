"""The activation rounding of the batch kernels that hold x in fp16 (the
sorted batch GEMM, the matrix-core small-M GEMM per K split): per row, fp16
of x * 2^e with the row maximum in [2^14, 2^15), scaled back exactly; fp16
activations are held as they are.  Tests feed the oracle this rounded
activation to pin the kernels' arithmetic to 1e-5."""
import numpy as np


def fp16_row_scaled(x: np.ndarray) -> np.ndarray:
    x = np.atleast_2d(np.asarray(x, dtype=np.float32))
    out = np.empty_like(x)
    for b in range(x.shape[0]):
        m = float(np.max(np.abs(x[b])))
        e = 14 - int(np.floor(np.log2(m))) if 0 < m < np.inf else 0
        out[b] = np.ldexp(np.ldexp(x[b], e).astype(np.float16).astype(np.float32), -e)
    return out
