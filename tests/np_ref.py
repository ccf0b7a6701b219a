"""Independent numpy restatement of the path's arithmetic, used only to
cross-check the C oracle. Written from the format definitions (GGUF K-quant
block layouts, the reference's symmetric quantiser in
crates/rocknpu-capi/src/lib.rs:614-654) without sharing code with oracle.c:
vectorised over whole blocks, scale fields unpacked bit-by-bit, rounding
implemented from floor/abs rather than roundf."""
import numpy as np

QK = 256


def f16(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32).reshape(-1)


def unpack_k4_scales(s: np.ndarray):
    """Twelve bytes -> eight 6-bit scales and mins, bit by bit: scale j<4 is
    bits 0-5 of byte j; min j<4 bits 0-5 of byte j+4; scale j>=4 takes its low
    nibble from byte j+4 and bits 4-5 from bits 6-7 of byte j-4; min j>=4 takes
    its low nibble from the high nibble of byte j+4 and bits 4-5 from bits 6-7
    of byte j."""
    s = s.astype(np.int32)
    sc = np.zeros((s.shape[0], 8), np.int32)
    mn = np.zeros((s.shape[0], 8), np.int32)
    for j in range(8):
        if j < 4:
            sc[:, j] = s[:, j] % 64
            mn[:, j] = s[:, j + 4] % 64
        else:
            sc[:, j] = (s[:, j + 4] % 16) + 16 * (s[:, j - 4] // 64)
            mn[:, j] = (s[:, j + 4] // 16) + 16 * (s[:, j] // 64)
    return sc, mn


def q4_k_ints(blocks: np.ndarray):
    """-> (d, dmin, sc[8], mn[8], q[256]) per block; q in value order."""
    b = blocks.reshape(-1, 144)
    d, dmin = f16(b[:, 0:2]), f16(b[:, 2:4])
    sc, mn = unpack_k4_scales(b[:, 4:16])
    qs = b[:, 16:].astype(np.int32).reshape(-1, 4, 32)
    q = np.concatenate([qs % 16, qs // 16], axis=2).reshape(-1, 256)  # per 64-chunk: lows then highs
    return d, dmin, sc, mn, q


def dequant_q4_k(blocks: np.ndarray) -> np.ndarray:
    d, dmin, sc, mn, q = q4_k_ints(blocks)
    sub = np.arange(256) // 32
    a = (d[:, None] * sc[:, sub].astype(np.float32)) * q.astype(np.float32)
    return (a - dmin[:, None] * mn[:, sub].astype(np.float32)).astype(np.float32)


def dequant_q5_k(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 176)
    d, dmin = f16(b[:, 0:2]), f16(b[:, 2:4])
    sc, mn = unpack_k4_scales(b[:, 4:16])
    qh = b[:, 16:48].astype(np.int32)
    qs = b[:, 48:].astype(np.int32).reshape(-1, 4, 32)
    q = np.empty((b.shape[0], 256), np.int32)
    for j in range(4):
        q[:, 64 * j:64 * j + 32] = qs[:, j] % 16 + 16 * ((qh >> (2 * j)) & 1)
        q[:, 64 * j + 32:64 * j + 64] = qs[:, j] // 16 + 16 * ((qh >> (2 * j + 1)) & 1)
    sub = np.arange(256) // 32
    a = (d[:, None] * sc[:, sub].astype(np.float32)) * q.astype(np.float32)
    return (a - dmin[:, None] * mn[:, sub].astype(np.float32)).astype(np.float32)


def q6_k_ints(blocks: np.ndarray):
    """-> (d, sc[16], q[256] in [-32, 31]) per block, q in value order."""
    b = blocks.reshape(-1, 210)
    ql = b[:, 0:128].astype(np.int32)
    qh = b[:, 128:192].astype(np.int32)
    sc = b[:, 192:208].view(np.int8).astype(np.int32)
    d = f16(b[:, 208:210])
    q = np.empty((b.shape[0], 256), np.int32)
    for p in range(256):
        half, r = divmod(p, 128)
        quarter, l = divmod(r, 32)
        byte = ql[:, 64 * half + l + 32 * (quarter % 2)]
        low = byte % 16 if quarter < 2 else byte // 16
        high = (qh[:, 32 * half + l] >> (2 * quarter)) & 3
        q[:, p] = low + 16 * high - 32
    return d, sc, q


def dequant_q6_k(blocks: np.ndarray) -> np.ndarray:
    d, sc, q = q6_k_ints(blocks)
    sub = np.arange(256) // 16
    return ((d[:, None] * sc[:, sub].astype(np.float32)) * q.astype(np.float32)).astype(np.float32)


def dequant(kind, blocks, n, k):
    f = {4: dequant_q4_k, 5: dequant_q5_k, 6: dequant_q6_k}[kind]
    return f(blocks).reshape(n, k)


def round_half_away(r: np.ndarray) -> np.ndarray:
    a = np.abs(r)
    f = np.floor(a)
    up = (a - f) >= np.float32(0.5)
    return np.sign(r) * (f + up)


def quantize_symmetric(rows: np.ndarray):
    rows = rows.astype(np.float32)
    mx = np.max(np.abs(rows), axis=1)
    scale = np.where(mx == 0, np.float32(1.0), mx / np.float32(127.0)).astype(np.float32)
    r = (rows / scale[:, None]).astype(np.float32)
    q = np.clip(round_half_away(r), -127, 127).astype(np.int8)
    return q, scale


def quantize_q8_k(x: np.ndarray):
    """-> (d [nb] f32, qs [nb,256] int32, bsums [nb,16] int32) for one row."""
    xb = x.astype(np.float32).reshape(-1, 256)
    idx = np.argmax(np.abs(xb), axis=1)                   # first largest magnitude
    mx = xb[np.arange(xb.shape[0]), idx]
    d = np.zeros(xb.shape[0], np.float32)
    qs = np.zeros(xb.shape, np.int32)
    nz = mx != 0
    iscale = (np.float32(-127.0) / mx[nz]).astype(np.float32)
    qs[nz] = np.minimum(127, np.rint((iscale[:, None] * xb[nz]).astype(np.float32))).astype(np.int32)
    d[nz] = (np.float32(1.0) / iscale).astype(np.float32)
    bsums = qs.reshape(-1, 16, 16).sum(axis=2)
    return d, qs, bsums


def pack_q8_k(d, qs, bsums) -> np.ndarray:
    out = np.zeros((d.size, 292), np.uint8)
    out[:, 0:4] = d.astype(np.float32).view(np.uint8).reshape(-1, 4)
    out[:, 4:260] = qs.astype(np.int8).view(np.uint8)
    out[:, 260:292] = bsums.astype(np.int16).view(np.uint8).reshape(-1, 32)
    return out.reshape(-1)


def block_sums(kind, w: np.ndarray, n: int, k: int, x: np.ndarray):
    """Exact per-(row, block) integer sums and the f64 row result."""
    nb = k // QK
    dq, qs, bs = quantize_q8_k(x)
    if kind == 4:
        d, dmin, sc, mn, q = q4_k_ints(w)
        sub = np.arange(256) // 32
        prod = q.reshape(n, nb, 256) * qs[None, :, :] * sc.reshape(n, nb, 8)[:, :, sub]
        isum = prod.sum(axis=2)
        pair = bs.reshape(nb, 8, 2).sum(axis=2)
        msum = (mn.reshape(n, nb, 8) * pair[None]).sum(axis=2)
        y = (d.reshape(n, nb).astype(np.float64) * dq[None] * isum -
             dmin.reshape(n, nb).astype(np.float64) * dq[None] * msum).sum(axis=1)
    else:
        d, sc, q = q6_k_ints(w)
        sub = np.arange(256) // 16
        prod = q.reshape(n, nb, 256) * qs[None, :, :] * sc.reshape(n, nb, 16)[:, :, sub]
        isum = prod.sum(axis=2)
        msum = np.zeros_like(isum)
        y = (d.reshape(n, nb).astype(np.float64) * dq[None] * isum).sum(axis=1)
    return isum.astype(np.int32), msum.astype(np.int32), y


def source_sample_fnv1a64(raw: bytes) -> int:
    """W8 sidecar fingerprint, restated from the generator
    (scripts/make_tinyllama_w8_sidecar_gguf.py:23-45) in plain Python."""
    mask = (1 << 64) - 1
    h = 14695981039346656037
    count = len(raw)
    for shift in range(0, 64, 8):
        h ^= (count >> shift) & 0xFF
        h = (h * 1099511628211) & mask
    sample = 4096
    if count <= sample * 3:
        ranges = ((0, count),)
    else:
        ranges = ((0, sample), ((count - sample) // 2, sample), (count - sample, sample))
    for start, n in ranges:
        for v in raw[start:start + n]:
            h ^= v
            h = (h * 1099511628211) & mask
    return h


def tie_rows(kind: int, n: int, k: int, seed: int) -> np.ndarray:
    """K-quant rows whose symmetric scale is a power of two, so that many
    v / scale land exactly on half-integers, where rounding half to even and
    half away from zero differ on every other one.
    Q4_K/Q5_K: d = 1/4, dmin = 127/64, sub-block 0 of each block has scale 1
    and min 32 (values q/4 - 63.5, the row's largest magnitude 63.5 at q = 0,
    placed in block 0), the other sub-blocks scales 1..16 (Q5_K 1..8) and min 0: scale
    0.5, v / scale = sc * q / 2. Q6_K: d = 1, sub-block 0 has scale 127 and a
    quant of -32 at value 0 (magnitude 4064), the others odd scales 1..61:
    scale 32, v / scale = sc * q / 32, a tie wherever q = +-16."""
    g = np.random.default_rng(seed)
    nbt = n * (k // QK)
    bb = {4: 144, 5: 176, 6: 210}[kind]
    blk = np.empty((nbt, bb), np.uint8)
    if kind in (4, 5):
        from rocknpu_amd import synth
        blk[:, 0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
        blk[:, 2:4] = np.frombuffer(np.float16(127 / 64).tobytes(), np.uint8)
        sc = g.integers(1, 17 if kind == 4 else 9, (nbt, 8))  # |d sc q| <= 60 / 62 < 63.5
        mn = np.zeros((nbt, 8), np.int64)
        sc[:, 0] = 1
        mn[:, 0] = 32
        blk[:, 4:16] = synth.pack_scales_k4(sc, mn)
        blk[:, 16:] = g.integers(0, 256, (nbt, bb - 16), dtype=np.uint8)
        blk = blk.reshape(n, -1, bb)
        # value 0 of block 0: low nibble of the first quant byte (and its Q5_K high bit) zero
        blk[:, 0, 16 if kind == 4 else 48] &= 0xF0
        if kind == 5:
            blk[:, 0, 16] &= 0xFE
    else:
        blk[:, 0:192] = g.integers(0, 256, (nbt, 192), dtype=np.uint8)
        sc = (2 * g.integers(0, 31, (nbt, 16)) + 1).astype(np.int8)
        sc[:, 0] = 127
        blk[:, 192:208] = sc.view(np.uint8)
        blk[:, 208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        blk = blk.reshape(n, -1, bb)
        blk[:, 0, 0] &= 0xF0    # value 0: low nibble 0
        blk[:, 0, 128] &= 0xFC  # and high bits 0, so q = -32
    return np.ascontiguousarray(blk.reshape(-1))


def tile_weights(kind: int, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """The decode cache's tile-interleaved copy of n rows of k/256 blocks,
    built with array reshapes (no per-byte index arithmetic): tiles of 16 rows
    (zero rows past n), each tile's blocks in order, and for tile t, block b:
    Q4_K: the 16 rows' 16-byte headers, then for lane l = 16 q + r the quant
    bytes 32 j + 8 q .. + 7 of row r, j = 0..3;
    Q6_K: the 16 rows' 16 scale bytes, their 2-byte d, then for lane
    l = 16 q + r the ql runs 64 h + 32 i + 8 q (order 2 h + i) and the qh runs
    128 + 32 h + 8 q, 8 bytes each."""
    bb = 144 if kind == 4 else 210
    nb = k // QK
    tiles = -(-n // 16)
    b = np.zeros((tiles * 16, nb, bb), np.uint8)
    b[:n] = blocks.reshape(n, nb, bb)
    b = b.reshape(tiles, 16, nb, bb).transpose(0, 2, 1, 3)  # [tile][block][row][byte]
    if kind == 4:
        head = b[..., :16].reshape(tiles, nb, 256)
        qs = b[..., 16:].reshape(tiles, nb, 16, 4, 4, 8)         # [row][j][q][8]
        lanes = qs.transpose(0, 1, 4, 2, 3, 5).reshape(tiles, nb, 2048)  # [q][row][j][8]
        out = np.concatenate([head, lanes], axis=2)
    else:
        sc = b[..., 192:208].reshape(tiles, nb, 256)
        d = b[..., 208:210].reshape(tiles, nb, 32)
        ql = b[..., :128].reshape(tiles, nb, 16, 2, 2, 4, 8)     # [row][h][i][q][8]
        ql = ql.transpose(0, 1, 5, 2, 3, 4, 6).reshape(tiles, nb, 4, 16, 32)  # [q][row][h i 8]
        qh = b[..., 128:192].reshape(tiles, nb, 16, 2, 4, 8)     # [row][h][q][8]
        qh = qh.transpose(0, 1, 4, 2, 3, 5).reshape(tiles, nb, 4, 16, 16)     # [q][row][h 8]
        lanes = np.concatenate([ql, qh], axis=4).reshape(tiles, nb, 3072)
        out = np.concatenate([sc, d, lanes], axis=2)
    return np.ascontiguousarray(out).reshape(-1)
