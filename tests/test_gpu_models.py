"""Model-shape MUL_MAT sequences at full size on the GPU, against the oracle.

Random-init Q4_K_M-style weights (Q4_K, with Q6_K for ffn_down and the output
head) of three architectures:
  TinyLlama-1.1B  22 layers, hidden 2048, FFN 5632, K/V 4 x 64,  vocab 32000
  Llama-3.2-1B    16 layers, hidden 2048, FFN 8192, K/V 8 x 64,  vocab 128256 (tied head)
  Llama-3-8B      32 layers, hidden 4096, FFN 14336, K/V 8 x 128, vocab 128256
Every MUL_MAT node of a prefill (all layers and the head) goes through
rocknpu_route_run in one call, as the ggml backend's graph_compute would hand
them over; each node's output is checked bit for bit against the oracle's W8A8
route on sampled activation rows (rows are independent: per-token quantisation,
one i32 dot product per output). The launch layer's repack and int32
accumulators are checked bit-exact on the largest shapes (the 128256 x 2048 Q6_K
head, the Llama-3-8B 128256 x 4096 Q6_K head, the 4096 x 14336 x 4096 GEMM) on
sampled row blocks. Batched decode on every Llama-3-8B projection (q/k/v, o,
gate+up, the Q6_K down) runs through both routes: W8A8 (exact) and the Q8_K
GEMV (within 1e-5 of the sum of the block terms' magnitudes, and of max |y|
per row).

Activations of the nodes are distinct windows of one random pool (distinct
pointers, as distinct graph tensors are), so the routing groups only what a
real graph would group: q/k/v and gate/up of one layer.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rocknpu_amd import hip
from rocknpu_amd import route as R
from rocknpu_amd import synth
from rocknpu_amd.capi import STATUS_OK, Context

pytestmark = pytest.mark.gpu

THREADS = 8
TYPE = {4: R.Q4_K, 6: R.Q6_K}
MODELS = {
    # layers, hidden, ffn, k/v rows, vocab
    "tinyllama": (22, 2048, 5632, 256, 32000),
    "llama32_1b": (16, 2048, 8192, 512, 128256),
    "llama3_8b": (32, 4096, 14336, 1024, 128256),
}


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def _layer_spec(hidden, ffn, kv):
    """(tensor, kind, n, k, input) in graph order."""
    return [("attn_q", 4, hidden, hidden, "attn"), ("attn_k", 4, kv, hidden, "attn"),
            ("attn_v", 4, kv, hidden, "attn"), ("attn_output", 4, hidden, hidden, "o"),
            ("ffn_gate", 4, ffn, hidden, "ffn"), ("ffn_up", 4, ffn, hidden, "ffn"),
            ("ffn_down", 6, hidden, ffn, "down")]


def _sample_rows(m, count, seed):
    if m <= count:
        return np.arange(m)
    g = np.random.default_rng(seed)
    inner = g.choice(np.arange(1, m - 1), size=count - 2, replace=False)
    return np.sort(np.concatenate([[0, m - 1], inner]))


class _Pool:
    """Activation windows [m, k] at distinct offsets of one random f32 pool."""

    def __init__(self, m, k_max, windows, seed):
        self.m, self.k_max = m, k_max
        self.data = synth.activations(1, m * k_max + 16 * windows, index=seed).reshape(-1)
        self.next = 0

    def take(self, k):
        off = 16 * self.next  # 64-byte steps: distinct, aligned pointers
        self.next += 1
        return self.data[off:off + self.m * k].reshape(self.m, k)


def _weights(model, layers, seed):
    n_layers, hidden, ffn, kv, vocab = MODELS[model]
    spec = _layer_spec(hidden, ffn, kv)
    ws = {}
    for layer in range(layers):
        for j, (name, kind, n, k, _) in enumerate(spec):
            ws[(layer, name)] = synth.kquant(kind, n, k, index=seed + 16 * layer + j)
    return spec, ws


def _check_w8a8_rows(kind, blocks, k, n, act, out, rows, what):
    w8, wsc = orc.repack_w8(kind, blocks, k, n, threads=THREADS)
    a8, asc = orc.quantize_a8(act[rows])
    ref = orc.rescale(orc.gemm_i32(a8, w8, threads=THREADS), asc, wsc)
    got = out[rows]
    assert np.array_equal(_bits(got), _bits(ref)), f"{what}: {np.sum(_bits(got) != _bits(ref))} outputs differ"


def _prefill_sequence(model, m, layers, head, seed):
    """All MUL_MAT nodes of `layers` layers (+ the head) through one
    rocknpu_route_run call; each checked on sampled rows."""
    n_layers, hidden, ffn, kv, vocab = MODELS[model]
    spec, ws = _weights(model, layers, seed)
    head_w = synth.kquant(6, vocab, hidden, index=seed + 9999) if head else None
    pool = _Pool(m, max(hidden, ffn), 4 * layers + 1, seed + 1)
    nodes, checks = [], []
    for layer in range(layers):
        acts = {tag: pool.take(ffn if tag == "down" else hidden) for tag in ("attn", "o", "ffn", "down")}
        for name, kind, n, k, tag in spec:
            out = np.full((m, n), np.nan, np.float32)
            w = ws[(layer, name)]
            nodes.append(R.node(TYPE[kind], w, k, n, acts[tag], out, name=f"blk.{layer}.{name}.weight"))
            checks.append((kind, w, k, n, acts[tag], out, f"{model} M={m} blk.{layer}.{name}"))
    if head:
        act = pool.take(hidden)
        out = np.full((m, vocab), np.nan, np.float32)
        nodes.append(R.node(R.Q6_K, head_w, hidden, vocab, act, out, name="output.weight"))
        checks.append((6, head_w, hidden, vocab, act, out, f"{model} M={m} output"))
    print(f"{model} prefill M={m}: {len(nodes)} nodes through rocknpu_route_run", flush=True)
    with Context() as ctx:
        assert R.run(ctx, nodes, R.DECODE_GGML) == STATUS_OK
        st = R.stats(ctx)
    rows = _sample_rows(m, 8, seed + 2)
    for kind, w, k, n, act, out, what in checks:
        _check_w8a8_rows(kind, w, k, n, act, out, rows, what)
    return st


@pytest.mark.parametrize("m", [128, 512])
def test_tinyllama_prefill_sequence_with_head(m):
    """TinyLlama-1.1B: the 22 layers' 154 projections and the 32000 x 2048 Q6_K head."""
    st = _prefill_sequence("tinyllama", m, 22, True, seed=40000 + m)
    print(st, flush=True)


def test_tinyllama_decode_step_with_head():
    """One decode step (M = 1) of TinyLlama-1.1B through the routing's GGML decode
    route (Q8_K activations, the GEMV), every layer and the head, against the
    oracle's ggml dot product."""
    _, hidden, ffn, kv, vocab = MODELS["tinyllama"]
    spec, ws = _weights("tinyllama", 22, 41000)
    head_w = synth.kquant(6, vocab, hidden, index=41999)
    pool = _Pool(1, ffn, 4 * 22 + 1, 41001)
    nodes, checks = [], []
    for layer in range(22):
        acts = {tag: pool.take(ffn if tag == "down" else hidden) for tag in ("attn", "o", "ffn", "down")}
        for name, kind, n, k, tag in spec:
            out = np.full((1, n), np.nan, np.float32)
            nodes.append(R.node(TYPE[kind], ws[(layer, name)], k, n, acts[tag], out))
            checks.append((kind, ws[(layer, name)], k, n, acts[tag], out))
    act = pool.take(hidden)
    out = np.full((1, vocab), np.nan, np.float32)
    nodes.append(R.node(R.Q6_K, head_w, hidden, vocab, act, out))
    checks.append((6, head_w, hidden, vocab, act, out))
    with Context() as ctx:
        assert R.run(ctx, nodes, R.DECODE_GGML) == STATUS_OK
    worst = 0.0
    for kind, w, k, n, act, out in checks:
        q8 = orc.quantize_q8_k(act)
        ref = orc.gemv_q8_k(kind, w, k, n, q8, threads=THREADS)[0]
        _, _, mag = orc.gemv_block_sums(kind, w, k, n, q8[0])
        err = np.abs(out[0].astype(np.float64) - ref)
        assert np.all(err <= 1e-5 * mag), (kind, n, k)
        worst = max(worst, float(err.max() / np.abs(ref).max()))
    print(f"decode step: max |err| / max |y| = {worst:.3g}", flush=True)
    assert worst <= 1e-5


@pytest.mark.parametrize("m", [128, 512, 2048])
def test_llama32_1b_prefill_sequence_with_tied_head(m):
    """Llama-3.2-1B: 16 layers (FFN 8192) and the tied 128256 x 2048 Q6_K output
    head through one routing call."""
    _prefill_sequence("llama32_1b", m, 16, True, seed=42000 + m)


def test_llama32_1b_head_repack_and_i32_exact():
    """The 128256 x 2048 Q6_K head: the GPU repack bit-exact against the oracle's
    (every row), A8 quantisation of 2048 tokens bit-exact, and the head GEMM's
    int32 accumulators and f32 outputs exact on 64 sampled rows."""
    vocab, hidden, m = 128256, 2048, 2048
    blocks = synth.kquant(6, vocab, hidden, index=43000)
    a = synth.activations(m, hidden, index=43001)
    print("head repack", flush=True)
    w8, wsc = hip.repack_w8(6, torch.from_numpy(blocks).to("cuda"), hidden, vocab)
    a8, asc = hip.quantize_a8(torch.from_numpy(a).to("cuda"))
    c = torch.empty((m, vocab), dtype=torch.int32, device="cuda")
    out = hip.gemm_w8a8(a8, asc, w8, wsc, out_i32=c)
    torch.cuda.synchronize()
    rw8, rsc = orc.repack_w8(6, blocks, hidden, vocab, threads=THREADS)
    assert np.array_equal(w8.cpu().numpy(), rw8)
    assert np.array_equal(_bits(wsc.cpu().numpy()), _bits(rsc))
    ra8, ras = orc.quantize_a8(a)
    assert np.array_equal(a8.cpu().numpy(), ra8)
    assert np.array_equal(_bits(asc.cpu().numpy()), _bits(ras))
    rows = _sample_rows(m, 64, 43002)
    rc = orc.gemm_i32(ra8[rows], rw8, threads=THREADS)
    assert np.array_equal(c[torch.from_numpy(rows).to("cuda")].cpu().numpy(), rc)
    assert np.array_equal(_bits(out[torch.from_numpy(rows).to("cuda")].cpu().numpy()),
                          _bits(orc.rescale(rc, ras[rows], rsc)))


@pytest.mark.parametrize("kind,n,k", [(4, 14336, 4096), (6, 4096, 14336)])
def test_llama3_8b_prefill_4096_gemm_i32_exact(kind, n, k):
    """Llama-3-8B at 4096 tokens: the gate (Q4_K 14336 x 4096) and down (Q6_K
    4096 x 14336) GEMMs, int32 accumulators exact on four 16-row blocks (one per
    quarter of M, so every tile row band of the large-tile kernel is sampled)."""
    m = 4096
    blocks = synth.kquant(kind, n, k, index=44000 + kind)
    a = synth.activations(m, k, index=44001 + kind)
    print(f"llama3-8b gemm kind={kind} n={n} k={k}", flush=True)
    w8, wsc = hip.repack_w8(kind, torch.from_numpy(blocks).to("cuda"), k, n)
    a8, asc = hip.quantize_a8(torch.from_numpy(a).to("cuda"))
    c = torch.empty((m, n), dtype=torch.int32, device="cuda")
    out = hip.gemm_w8a8(a8, asc, w8, wsc, out_i32=c)
    torch.cuda.synchronize()
    g = np.random.default_rng(44002)
    rows = np.concatenate([np.arange(b, b + 16) for b in
                           [0] + [q * 1024 + 16 * int(g.integers(0, 64)) for q in (1, 2)] + [m - 16]])
    rw8, rsc = orc.repack_w8(kind, blocks, k, n, threads=THREADS)
    ra8, ras = orc.quantize_a8(a[rows])
    rc = orc.gemm_i32(ra8, rw8, threads=THREADS)
    idx = torch.from_numpy(rows).to("cuda")
    assert np.array_equal(c[idx].cpu().numpy(), rc)
    assert np.array_equal(_bits(out[idx].cpu().numpy()), _bits(orc.rescale(rc, ras, rsc)))


def test_llama3_8b_head_repack_and_i32_exact():
    """The Llama-3-8B output head (Q6_K 128256 x 4096, the vocabulary head the
    reference leaves on the CPU, ggml-rocknpu.cpp:644-650): the GPU repack
    bit-exact against the oracle's on every row, and the 4096-token GEMM's int32
    accumulators and f32 outputs exact on four 16-row blocks (one per quarter
    of M)."""
    vocab, hidden, m = 128256, 4096, 4096
    blocks = synth.kquant(6, vocab, hidden, index=47000)
    a = synth.activations(m, hidden, index=47001)
    print("llama3-8b head repack", flush=True)
    w8, wsc = hip.repack_w8(6, torch.from_numpy(blocks).to("cuda"), hidden, vocab)
    a8, asc = hip.quantize_a8(torch.from_numpy(a).to("cuda"))
    c = torch.empty((m, vocab), dtype=torch.int32, device="cuda")
    out = hip.gemm_w8a8(a8, asc, w8, wsc, out_i32=c)
    torch.cuda.synchronize()
    rw8, rsc = orc.repack_w8(6, blocks, hidden, vocab, threads=THREADS)
    assert np.array_equal(w8.cpu().numpy(), rw8)
    assert np.array_equal(_bits(wsc.cpu().numpy()), _bits(rsc))
    del blocks
    g = np.random.default_rng(47002)
    rows = np.concatenate([np.arange(b, b + 16) for b in
                           [0] + [q * 1024 + 16 * int(g.integers(0, 64)) for q in (1, 2)] + [m - 16]])
    ra8, ras = orc.quantize_a8(a[rows])
    idx = torch.from_numpy(rows).to("cuda")
    assert np.array_equal(a8[idx].cpu().numpy(), ra8)
    rc = orc.gemm_i32(ra8, rw8, threads=THREADS)
    assert np.array_equal(c[idx].cpu().numpy(), rc)
    assert np.array_equal(_bits(out[idx].cpu().numpy()), _bits(orc.rescale(rc, ras, rsc)))


def test_llama3_8b_prefill_layer_sequence():
    """Llama-3-8B at 4096 tokens: two layers' projections (q/k/v grouped, o,
    gate/up grouped, down) through one routing call, sampled rows exact."""
    _prefill_sequence("llama3_8b", 4096, 2, False, seed=45000)


# Llama-3-8B decode projections: (name, kinds, rows per member, K)
L3_DECODE = {
    "qkv": ((4, 4, 4), (4096, 1024, 1024), 4096),
    "o": ((4,), (4096,), 4096),
    "gate_up": ((4, 4), (14336, 14336), 4096),
    "down": ((6,), (4096,), 14336),
}


@pytest.mark.parametrize("proj", list(L3_DECODE))
@pytest.mark.parametrize("m", [1, 8, 32, 64])
def test_llama3_8b_batched_decode_both_routes(proj, m):
    """Decode at batch 1, 8, 32, 64 on every Llama-3-8B projection (q/k/v and
    gate+up as one call each, o, and the Q6_K down): the W8A8 route (concat
    call) and the Q8_K GEMV route (grouped call, the decode cache's tiled
    copies from two rows), on sampled rows: the first exact, the second within
    1e-5 of the block terms' magnitude and of max |y| per row."""
    kinds, ns, k = L3_DECODE[proj]
    ws = [synth.kquant(kind, n, k, index=46000 + 10 * list(L3_DECODE).index(proj) + i)
          for i, (kind, n) in enumerate(zip(kinds, ns))]
    x = synth.activations(m, k, index=46010 + m + k)
    print(f"llama3-8b batched decode {proj} m={m}", flush=True)
    with Context() as ctx:
        w8a8 = [np.full((m, n), np.nan, np.float32) for n in ns]
        assert ctx.matmul_q_concat(ws, list(kinds), list(ns), x, w8a8, k) == STATUS_OK
        q8route = [np.full((m, n), np.nan, np.float32) for n in ns]
        assert ctx.matmul_q_q8k_group(ws, list(kinds), list(ns), x, q8route, k) == STATUS_OK
    rows = _sample_rows(m, 8, 46020 + m)
    q8 = orc.quantize_q8_k(x[rows])
    worst = 0.0
    for kind, n, w, o1, o2 in zip(kinds, ns, ws, w8a8, q8route):
        _check_w8a8_rows(kind, w, k, n, x, o1, rows, f"w8a8 {proj} m={m}")
        ref = orc.gemv_q8_k(kind, w, k, n, q8, threads=THREADS)
        for i, mi in enumerate(rows):
            _, _, mag = orc.gemv_block_sums(kind, w, k, n, q8[i])
            err = np.abs(o2[mi].astype(np.float64) - ref[i])
            assert np.all(err <= 1e-5 * mag), (proj, mi)
            worst = max(worst, float(err.max() / np.abs(ref[i]).max()))
    print(f"q8k route {proj} m={m}: max |err| / max |y| = {worst:.3g}", flush=True)
    assert worst <= 1e-5
