"""The W8 sidecar on the CPU: the provenance fingerprint against published
FNV-1a vectors, the oracle and a plain-Python restatement of the generator;
the three files written and read byte for byte by the library (host code,
no device work); every rejection the reader applies."""
import os

import numpy as np
import pytest

from oracle import oracle as orc
from rocknpu_amd import sidecar, synth

from . import np_ref

SIZES = [1, 7, 4096, 12287, 12288, 12289, 12290, 20001, 144 * 88]


def test_fnv1a64_published_vectors():
    # FNV-1a 64-bit test vectors (Fowler/Noll/Vo reference set)
    assert orc.fnv1a64(b"") == 0xcbf29ce484222325
    assert orc.fnv1a64(b"a") == 0xaf63dc4c8601ec8c
    assert orc.fnv1a64(b"foobar") == 0x85944171f73967e8


@pytest.mark.parametrize("size", SIZES)
def test_fingerprint_matches_oracle_and_restatement(size):
    data = np.random.default_rng(size).integers(0, 256, size, dtype=np.uint8)
    expect = np_ref.source_sample_fnv1a64(data.tobytes())
    assert orc.source_fingerprint(data) == expect
    assert sidecar.fingerprint(data) == expect


def test_fingerprint_samples_first_middle_last():
    size = 50001
    data = np.random.default_rng(1).integers(0, 256, size, dtype=np.uint8)
    base = sidecar.fingerprint(data)
    mid = (size - 4096) // 2
    for pos, counted in ((0, True), (4095, True), (4096, False), (mid - 1, False), (mid, True), (mid + 4095, True),
                         (mid + 4096, False), (size - 4097, False), (size - 4096, True), (size - 1, True)):
        d = data.copy()
        d[pos] ^= 0x5A
        assert (sidecar.fingerprint(d) != base) == counted, pos
    # a planted mistake in the middle window (starting at the centre instead of
    # centring the window) is caught
    raw = data.tobytes()
    h = 14695981039346656037
    for shift in range(0, 64, 8):
        h = ((h ^ ((size >> shift) & 0xFF)) * 1099511628211) & ((1 << 64) - 1)
    for start in (0, size // 2, size - 4096):  # planted: size/2 instead of (size - 4096)/2
        for v in raw[start:start + 4096]:
            h = ((h ^ v) * 1099511628211) & ((1 << 64) - 1)
    assert h != base


def _tensor(n=24, k=512, seed=3):
    blocks = synth.q4_k(n, k, index=seed)
    w8 = np.random.default_rng(seed).integers(-127, 128, (n, k), dtype=np.int8)
    scales = (np.random.default_rng(seed + 1).random(n, dtype=np.float32) + np.float32(0.01)) / np.float32(127)
    return blocks, w8, scales


def test_write_then_read_round_trip(tmp_path):
    blocks, w8, scales = _tensor()
    n, k = w8.shape
    assert sidecar.write(tmp_path, "blk.0.ffn_gate.weight", blocks, w8, scales) == 0
    base = tmp_path / "blk.0.ffn_gate.weight"
    assert (tmp_path / (base.name + ".w8")).read_bytes() == w8.tobytes()
    assert (tmp_path / (base.name + ".scale.f32")).read_bytes() == scales.astype("<f4").tobytes()
    assert (tmp_path / (base.name + ".source.fnv1a64")).read_text() == f"{np_ref.source_sample_fnv1a64(blocks.tobytes()):016x}\n"
    got = sidecar.read(tmp_path, "blk.0.ffn_gate.weight", blocks, k, n)
    assert got is not None
    assert np.array_equal(got[0], w8) and np.array_equal(got[1].view(np.uint32), scales.view(np.uint32))


def test_reader_accepts_generator_files(tmp_path):
    """Files laid out as the generator writes them (numpy tofile, hex digest and a newline;
    make_tinyllama_w8_sidecar_gguf.py:66-69,110-112), upper-case hex included."""
    blocks, w8, scales = _tensor(seed=5)
    n, k = w8.shape
    name = "blk.3.attn_q.weight"
    w8.tofile(tmp_path / f"{name}.w8")
    scales.tofile(tmp_path / f"{name}.scale.f32")
    (tmp_path / f"{name}.source.fnv1a64").write_text(f"{np_ref.source_sample_fnv1a64(blocks.tobytes()):016X}\n")
    got = sidecar.read(tmp_path, name, blocks, k, n)
    assert got is not None and np.array_equal(got[0], w8)


def test_reader_rejections(tmp_path):
    blocks, w8, scales = _tensor(seed=7)
    n, k = w8.shape
    name = "t"
    assert sidecar.write(tmp_path, name, blocks, w8, scales) == 0
    other = blocks.copy()
    other[5] ^= 1
    assert sidecar.read(tmp_path, name, other, k, n) is None             # source changed
    assert sidecar.read(tmp_path, name, blocks, k, n + 1) is None         # wrong shape: sizes differ
    assert sidecar.read(tmp_path, "missing", blocks, k, n) is None
    w = tmp_path / f"{name}.w8"
    data = w.read_bytes()
    w.write_bytes(data[:-1])
    assert sidecar.read(tmp_path, name, blocks, k, n) is None             # truncated weights
    w.write_bytes(data)
    bad = scales.copy()
    bad[3] = 0.0
    bad.tofile(tmp_path / f"{name}.scale.f32")
    assert sidecar.read(tmp_path, name, blocks, k, n) is None             # scale not > 0
    bad[3] = np.nan
    bad.tofile(tmp_path / f"{name}.scale.f32")
    assert sidecar.read(tmp_path, name, blocks, k, n) is None
    scales.tofile(tmp_path / f"{name}.scale.f32")
    fp = tmp_path / f"{name}.source.fnv1a64"
    good = fp.read_text()
    fp.write_text(good.strip()[:-1] + "\n")                               # 15 digits
    assert sidecar.read(tmp_path, name, blocks, k, n) is None
    fp.write_text(good.strip() + "x\n")
    assert sidecar.read(tmp_path, name, blocks, k, n) is None
    fp.write_text("  " + good.strip() + "  \n")                           # whitespace around is fine
    assert sidecar.read(tmp_path, name, blocks, k, n) is not None
    # the writer refuses non-positive scales
    assert sidecar.write(tmp_path, "u", blocks, w8, bad) == -1
    assert not os.path.exists(tmp_path / "u.w8")
