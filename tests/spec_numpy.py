"""An independent numpy restatement of the quantize spec and of the packed format.

Used only to cross-check the C oracle (a second implementation written from the
same specification: QuantizedTensor.kt:256-324 and the JDK contract of
Math.round). numpy float32 arithmetic is IEEE-754 binary32 with correct rounding
and gradual underflow, like the JVM's.
"""
from __future__ import annotations

import numpy as np

F32_MAX = np.float32(np.finfo(np.float32).max)


class RoundNaN(Exception):
    pass


def java_round(x: np.ndarray) -> np.ndarray:
    """Math.round for float32 arrays: nearest, ties toward +inf, saturating to int32.
    Raises RoundNaN if any element is NaN (Float.roundToInt rejects NaN)."""
    x = np.asarray(x, dtype=np.float32)
    if np.isnan(x).any():
        raise RoundNaN()
    xd = x.astype(np.float64)  # exact
    r = np.floor(xd + 0.5)     # exact in float64 for every float32
    r = np.clip(r, -2147483648.0, 2147483647.0)
    return r.astype(np.int64)


def wrap_i32(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, dtype=np.int64) & 0xFFFFFFFF
    return np.where(v >= 2**31, v - 2**32, v)


def quantize(data: np.ndarray, bits: int, group_size: int):
    """Returns (qdata uint8 [K*bpr], scales f32 [G*N], zeros int8 [G*N] or None)."""
    data = np.ascontiguousarray(data, dtype=np.float32)
    K, N = data.shape
    G = (K + group_size - 1) // group_size
    bpr = (N + N % 2) // 2 if bits == 4 else N
    scales = np.empty((G, N), dtype=np.float32)
    zeros = np.empty((G, N), dtype=np.int8) if bits == 4 else None
    qv = np.zeros((K, N), dtype=np.int64)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore", under="ignore"):
        for gi in range(G):
            blk = data[gi * group_size:(gi + 1) * group_size]
            if bits == 8:
                a = np.abs(blk)
                mx = np.where(np.isnan(a), np.float32(0), a).max(axis=0).astype(np.float32)
                scale = np.where(mx > 0, mx / np.float32(127.0), np.float32(1.0)).astype(np.float32)
                inv = (np.float32(1.0) / scale).astype(np.float32)
                q = java_round((blk * inv).astype(np.float32))
                qv[gi * group_size:gi * group_size + blk.shape[0]] = np.clip(q, -127, 127)
                scales[gi] = scale
            else:
                mn = np.where(np.isnan(blk), F32_MAX, blk).min(axis=0).astype(np.float32)
                mx = np.where(np.isnan(blk), -F32_MAX, blk).max(axis=0).astype(np.float32)
                mn = np.where(mn > 0, np.float32(0), mn).astype(np.float32)
                mx = np.where(mx < 0, np.float32(0), mx).astype(np.float32)
                rng = (mx - mn).astype(np.float32)
                scale = np.where(rng > 0, rng / np.float32(15.0), np.float32(1.0)).astype(np.float32)
                zero = np.clip(java_round((-mn / scale).astype(np.float32)), 0, 15)
                inv = (np.float32(1.0) / scale).astype(np.float32)
                q = wrap_i32(java_round((blk * inv).astype(np.float32)) + zero)
                qv[gi * group_size:gi * group_size + blk.shape[0]] = np.clip(q, 0, 15)
                scales[gi] = scale
                zeros[gi] = zero.astype(np.int8)
    if bits == 8:
        qdata = (qv & 0xFF).astype(np.uint8).reshape(-1)
    else:
        half = bpr
        packed = np.zeros((K, bpr), dtype=np.int64)
        packed[:, :half] |= qv[:, :half]
        high = qv[:, half:]
        packed[:, :high.shape[1]] |= high << 4
        qdata = packed.astype(np.uint8).reshape(-1)
    return qdata, scales.reshape(-1), None if zeros is None else zeros.reshape(-1)


def decode(qdata, scales, zeros, K, N, bits, group_size) -> np.ndarray:
    """fp32 [K x N] of value(r, c) = scale * (raw - zero) (QuantizedTensor.kt:172-186)."""
    bpr = (N + N % 2) // 2 if bits == 4 else N
    q = np.asarray(qdata).view(np.uint8).reshape(K, bpr)
    if bits == 8:
        raw = q.view(np.int8).astype(np.int32)
    else:
        half = bpr
        raw = np.empty((K, N), dtype=np.int32)
        raw[:, :half] = q[:, :half] & 0xF
        raw[:, half:] = (q[:, :N - half] >> 4) & 0xF
    G = (K + group_size - 1) // group_size
    gidx = np.arange(K) // group_size
    s = np.asarray(scales, dtype=np.float32).reshape(G, N)[gidx]
    if zeros is None:
        z = np.zeros((K, N), dtype=np.int32)
    else:
        z = np.asarray(zeros).view(np.int8).reshape(G, N)[gidx].astype(np.int32)
    return (s * (raw - z).astype(np.float32)).astype(np.float32)


def pack_column_runs(qdata, K: int, N: int, bits: int, scales=None, zeros=None, g: int = 0) -> np.ndarray:
    """The column-run copy (kt_qweight_pack), restated with numpy reshapes: the weight
    blocks, then (with scales and g given) the scale and zero-point rows and the trailer
    (the largest |scale|).

    Blocks [column set of 16][chunk of 128 k]; in a block, lane l = 16 kb + n owns 16
    bytes (INT8: two halves of 1 KB, lane bytes at h * 1024 + 16 l) for column 16 set + n
    and k in [128 chunk + 32 kb, + 32). INT8 byte b of half h is k = run + 16 h + b;
    INT4 byte 8 m + 4 hh + t holds k = run + 16 m + 8 hh + t (low nibble) and that k + 4
    (high nibble). Values outside [K x N] are 0."""
    bpr = (N + N % 2) // 2 if bits == 4 else N
    q = np.asarray(qdata).view(np.uint8).reshape(K, bpr)
    if bits == 8:
        vals = q[:, :N]
    else:
        vals = np.empty((K, N), dtype=np.uint8)
        vals[:, :bpr] = q[:, :bpr] & 0xF
        vals[:, bpr:] = (q[:, :N - bpr] >> 4) & 0xF
    sets, chunks = -(-N // 16), -(-K // 128)
    V = np.zeros((chunks * 128, sets * 16), dtype=np.uint8)
    V[:K, :N] = vals
    if bits == 8:
        R = V.reshape(chunks, 4, 2, 16, sets, 16)           # c, kb, h, b, set, n
        blocks = np.ascontiguousarray(R.transpose(4, 0, 2, 1, 5, 3)).reshape(-1)  # set, c, h, kb, n, b
    else:
        R = V.reshape(chunks, 4, 2, 2, 2, 4, sets, 16)      # c, kb, m, hh, lohi, t, set, n
        byte = R[:, :, :, :, 0] | (R[:, :, :, :, 1] << 4)   # c, kb, m, hh, t, set, n
        blocks = np.ascontiguousarray(byte.transpose(5, 0, 1, 6, 2, 3, 4)).reshape(-1)  # set, c, kb, n, m, hh, t
    if scales is None:
        return blocks
    # [set][group][16] rows: fp32 scales, then zero-point bytes (0 past N or without zeros)
    G = -(-K // g)
    S = np.zeros((G, sets * 16), dtype=np.float32)
    S[:, :N] = np.asarray(scales, dtype=np.float32).reshape(G, N)
    Z = np.zeros((G, sets * 16), dtype=np.uint8)
    if zeros is not None:
        Z[:, :N] = np.asarray(zeros).view(np.uint8).reshape(G, N)
    srows = np.ascontiguousarray(S.reshape(G, sets, 16).transpose(1, 0, 2)).view(np.uint8).reshape(-1)
    zrows = np.ascontiguousarray(Z.reshape(G, sets, 16).transpose(1, 0, 2)).reshape(-1)
    # the trailer: the largest |scale| (fmax: NaNs ignored), then 12 zero bytes
    trailer = np.zeros(4, dtype=np.float32)
    trailer[0] = np.fmax.reduce(np.abs(S.ravel()), initial=np.float32(0))
    return np.concatenate([blocks, srows, zrows, trailer.view(np.uint8)])
