"""GPU parity of the op-level kernels against the CPU oracle, through the C ABI.

Bars: i32 accumulators and int8 codes bit-exact; fp32 outputs within 1e-3
relative (the stated tolerance), and in practice bit-identical because the
kernels evaluate the oracle's canonical operation order — the strict tests
assert that too.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


@pytest.fixture(scope="module")
def dev(pkg):
    from importlib import import_module

    d = import_module(pkg.__name__ + ".device")
    assert d.device_count() >= 1, "no HIP device visible"
    print(f"device: {d.device_name(0)}", flush=True)
    return d


def rel_err(got, want):
    den = np.maximum(np.abs(want), 1e-6)
    return float(np.max(np.abs(got.astype(np.float64) - want) / den)) if got.size else 0.0


@pytest.mark.parametrize("K,N", [(512, 1536), (512, 512), (512, 2048), (2048, 512), (512, 32000)])
@pytest.mark.parametrize("M", [1, 8, 64, 256, 4096])
def test_q8_linear_sweep(pkg, orc, dev, M, K, N):
    print(f"q8_linear M={M} K={K} N={N}", flush=True)
    a, w, mult, bias = pkg.gemm_inputs(M, K, N)
    y_ref, acc_ref, q_ref, s_ref = orc.linear_forward(a, w, mult, bias, threads=16)
    da, dw, dm, db = (dev.DeviceArray.from_host(x) for x in (a, w, mult, bias))
    di = dev.DeviceArray.zeros((M, N), np.int32)
    df = dev.DeviceArray.zeros((M, N), np.float32)
    err = dev.DeviceArray.zeros(1, np.int32)
    dev.q8_linear(da, dw, dm, db, di, df, err=err)
    dev.synchronize()
    acc, y = di.host(), df.host()
    assert err.host()[0] == 0
    assert np.array_equal(acc, acc_ref), "i32 accumulators differ"
    assert rel_err(y, y_ref) <= REL_TOL
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), "dequant not bit-identical"


@pytest.mark.parametrize("K,N", [(2048, 512), (1536, 384)])
@pytest.mark.parametrize("M", [17, 33, 50, 64])
def test_q8_linear_long_k_row_groups(pkg, orc, dev, M, K, N):
    """fp32-only outputs above 16 rows at K = 1536 or 2048 run the skinny
    kernel with one 16-row group per workgroup (the decode FFN
    down-projection's path); ragged row counts leave a partial last group.
    Bit-identical to the oracle."""
    print(f"q8_linear row groups M={M} K={K} N={N}", flush=True)
    a, w, mult, bias = pkg.gemm_inputs(M, K, N)
    y_ref, _, _, _ = orc.linear_forward(a, w, mult, bias, threads=16)
    da, dw, dm, db = (dev.DeviceArray.from_host(x) for x in (a, w, mult, bias))
    df = dev.DeviceArray.zeros((M, N), np.float32)
    err = dev.DeviceArray.zeros(1, np.int32)
    dev.q8_linear(da, dw, dm, db, None, df, err=err)
    dev.synchronize()
    assert err.host()[0] == 0
    assert np.array_equal(df.host().view(np.uint32), y_ref.view(np.uint32))


def test_q8_linear_on_two_streams_at_once(pkg, orc, dev):
    """The op-level entry points keep their intermediate buffers (here the
    quantized activations of an fp32 input) per (device, stream): two streams
    that issue calls at the same time, with different row counts and no
    synchronization between them, each get the oracle's result bit for bit."""
    K, N = 512, 512
    shapes = {"a": 2048, "b": 96}
    print("q8_linear on two streams: rows " + ", ".join(map(str, shapes.values())), flush=True)
    w, mult, bias = None, None, None
    inputs, refs = {}, {}
    for i, (key, M) in enumerate(shapes.items()):
        a, w_i, mult_i, bias_i = pkg.gemm_inputs(M, K, N, seed=100 + i)
        if w is None:
            w, mult, bias = w_i, mult_i, bias_i
        inputs[key] = a
        refs[key] = orc.linear_forward(a, w, mult, bias, threads=16)[0]
    dw, dm, db = (dev.DeviceArray.from_host(x) for x in (w, mult, bias))
    streams = {k: dev.Stream() for k in shapes}
    try:
        din = {k: dev.DeviceArray.from_host(inputs[k]) for k in shapes}
        outs = {k: [dev.DeviceArray.zeros((shapes[k], N), np.float32) for _ in range(4)] for k in shapes}
        err = dev.DeviceArray.zeros(1, np.int32)
        for rep in range(4):  # interleaved, never waiting
            for k in shapes:
                dev.q8_linear(din[k], dw, dm, db, None, outs[k][rep], err=err, stream=streams[k].handle)
        for st in streams.values():
            st.sync()
        assert err.host()[0] == 0
        for k in shapes:
            for rep in range(4):
                assert np.array_equal(outs[k][rep].host().view(np.uint32), refs[k].view(np.uint32)), (k, rep)
    finally:
        for st in streams.values():
            st.close()


def test_quantize_rows_matches_oracle(pkg, orc, dev):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((300, 2048)) * rng.uniform(0.01, 50, size=(300, 1))).astype(np.float32)
    x[5] = 0.0  # all-zero row -> multiplier 1
    x[7, :10] = [0.5, 1.5, -0.5, -1.5, 2.5, -2.5, 126.5, 3.0, 0.0, -0.0]
    q_ref, a_ref = orc.quantize_rows(x)
    dx = dev.DeviceArray.from_host(x)
    dq = dev.DeviceArray.zeros(x.shape, np.int8)
    da = dev.DeviceArray.zeros(300, np.float32)
    err = dev.DeviceArray.zeros(1, np.int32)
    dev.quantize_rows(dx, dq, da, err)
    dev.synchronize()
    assert np.array_equal(dq.host(), q_ref) and np.array_equal(da.host(), a_ref)
    assert err.host()[0] == 0
    # a non-finite activation raises the error flag (the reference rejects it)
    x[3, 17] = np.inf
    dx2 = dev.DeviceArray.from_host(x)
    dev.quantize_rows(dx2, dq, da, err)
    dev.synchronize()
    assert err.host()[0] == 1


def test_q8_linear_edges(pkg, orc, dev):
    rng = np.random.default_rng(12)
    # column tail (N not a multiple of 16/64), odd M on both kernels, ReLU,
    # full-range weights including -128 (exact in the int8 matrix core); the
    # last two are wide grids (more than 64 column tiles) whose tiles go in
    # groups of eight row tiles, with a partial group and ragged edges
    for M, K, N in [(3, 64, 100), (77, 128, 130), (200, 192, 65), (130, 64, 1), (200, 64, 4170),
                    (610, 128, 4500)]:
        print(f"edge M={M} K={K} N={N}", flush=True)
        a = rng.standard_normal((M, K)).astype(np.float32)
        w = rng.integers(-128, 128, size=(N, K)).astype(np.int8)
        mult = rng.uniform(50, 100, size=N).astype(np.float32)
        bias = rng.standard_normal(N).astype(np.float32)
        y_ref, acc_ref, _, _ = orc.linear_forward(a, w, mult, bias, relu=True)
        dw = dev.DeviceArray.from_host(w)
        di = dev.DeviceArray.zeros((M, N), np.int32)
        df = dev.DeviceArray.zeros((M, N), np.float32)
        dev.q8_linear(dev.DeviceArray.from_host(a), dw, dev.DeviceArray.from_host(mult),
                      dev.DeviceArray.from_host(bias), di, df, relu=True)
        dev.synchronize()
        assert np.array_equal(di.host(), acc_ref)
        assert np.array_equal(df.host(), y_ref)
    # K not a multiple of 64 is rejected on the host
    with pytest.raises(RuntimeError):
        dev.q8_linear(dev.DeviceArray.zeros((2, 100), np.float32), dev.DeviceArray.zeros((4, 100), np.int8),
                      dev.DeviceArray.zeros(4, np.float32), dev.DeviceArray.zeros(4, np.float32),
                      dev.DeviceArray.zeros((2, 4), np.int32), None)


def test_residual_layer_norm_matches_oracle(pkg, orc, dev):
    rng = np.random.default_rng(13)
    for d in (512, 384):
        y = rng.standard_normal((257, d)).astype(np.float32)
        r = (rng.standard_normal((257, d)) * 3).astype(np.float32)
        g = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        b = (0.1 * rng.standard_normal(d)).astype(np.float32)
        ref = orc.residual_layer_norm(y, r, g, b)
        q_ref, a_ref = orc.quantize_rows(ref)
        out = dev.DeviceArray.zeros(y.shape, np.float32)
        q = dev.DeviceArray.zeros(y.shape, np.int8)
        a = dev.DeviceArray.zeros(257, np.float32)
        dev.residual_layer_norm(dev.DeviceArray.from_host(y), dev.DeviceArray.from_host(r),
                                dev.DeviceArray.from_host(g), dev.DeviceArray.from_host(b), out, q, a)
        dev.synchronize()
        assert np.array_equal(out.host(), ref)
        assert np.array_equal(q.host(), q_ref) and np.array_equal(a.host(), a_ref)


def _ln_edge_rows(rng, d=512):
    """Rows whose sequential sums stress the speculative folds (chunks of 64
    or 128):
    prefixes cancelling to near zero at the chunk boundaries (the candidate
    windows miss and chunks are refolded), exact zeros and negative zeros,
    constants, wide and tiny magnitudes."""
    rows = []
    for _ in range(8):  # cancellation at every 64-element chunk boundary
        z = rng.standard_normal(d).astype(np.float32) * np.float32(rng.uniform(0.5, 20))
        for k in range(64, d, 64):
            s = np.float32(-0.0)
            for v in z[:k - 1]:
                s = np.float32(s + v)
            z[k - 1] = -s + np.float32(rng.standard_normal() * 1e-5)
        rows.append(z)
    rows.append(np.zeros(d, np.float32))
    rows.append(np.full(d, -0.0, np.float32))
    rows.append(np.full(d, 0.3, np.float32))
    rows.append((rng.standard_normal(d) * 1e17).astype(np.float32))
    rows.append((rng.standard_normal(d) * 1e-39).astype(np.float32))  # subnormal
    alt = np.where(np.arange(d) % 2 == 0, 1e4, -1e4).astype(np.float32)
    rows.append(alt + (rng.standard_normal(d) * 1e-3).astype(np.float32))
    return np.stack(rows)


@pytest.mark.parametrize("d", [256, 384, 512])
def test_residual_layer_norm_single_wave_speculative_edges(pkg, orc, dev, d):
    """Rows of 256, 384 and 512 fold as two, three or four speculative
    128-element chunks inside one wave (the LayerNorms of both graphs):
    chunk boundaries where the prefix cancels to near zero force refolds; the
    result is the sequential fold's, bit for bit, and non-finite rows keep
    their NaN positions."""
    rng = np.random.default_rng(23 + d)
    z = np.concatenate([_ln_edge_rows(rng, d), rng.standard_normal((21, d)).astype(np.float32) * 3])
    y = (z * np.float32(0.75)).astype(np.float32)
    r = (z - y).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    b = (0.1 * rng.standard_normal(d)).astype(np.float32)
    ref = orc.residual_layer_norm(y, r, g, b)
    q_ref, a_ref = orc.quantize_rows(ref)
    out = dev.DeviceArray.zeros(y.shape, np.float32)
    q = dev.DeviceArray.zeros(y.shape, np.int8)
    a = dev.DeviceArray.zeros(y.shape[0], np.float32)
    dev.residual_layer_norm(dev.DeviceArray.from_host(y), dev.DeviceArray.from_host(r),
                            dev.DeviceArray.from_host(g), dev.DeviceArray.from_host(b), out, q, a)
    dev.synchronize()
    assert np.array_equal(out.host().view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(q.host(), q_ref) and np.array_equal(a.host(), a_ref)
    y2 = y[:3].copy()
    y2[0, 130] = np.nan
    y2[1, 257 % d] = np.inf
    y2[2, 5] = -np.inf
    ref2 = orc.residual_layer_norm(y2, r[:3], g, b)
    out2 = dev.DeviceArray.zeros(y2.shape, np.float32)
    err = dev.DeviceArray.zeros(1, np.int32)
    dev.residual_layer_norm(dev.DeviceArray.from_host(y2), dev.DeviceArray.from_host(r[:3]),
                            dev.DeviceArray.from_host(g), dev.DeviceArray.from_host(b), out2, err=err)
    dev.synchronize()
    got2 = out2.host()
    assert np.array_equal(np.isnan(got2), np.isnan(ref2))
    fin = ~np.isnan(ref2)
    assert np.array_equal(got2[fin], ref2[fin])
    assert err.host()[0] == 1


def test_residual_layer_norm_few_rows_edge_cases(pkg, orc, dev):
    """Rows of width 512 (four speculative 128-element chunks in one wave):
    the edge rows among ordinary ones, with their quantization."""
    rng = np.random.default_rng(17)
    z = _ln_edge_rows(rng)
    base = rng.standard_normal((48, 512)).astype(np.float32) * 2
    z = np.concatenate([z, base])
    y = (z * np.float32(0.75)).astype(np.float32)
    r = (z - y).astype(np.float32)  # y + r rounds back near z; the oracle sees the same y, r
    g = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    b = (0.1 * rng.standard_normal(512)).astype(np.float32)
    ref = orc.residual_layer_norm(y, r, g, b)
    q_ref, a_ref = orc.quantize_rows(ref)
    out = dev.DeviceArray.zeros(y.shape, np.float32)
    q = dev.DeviceArray.zeros(y.shape, np.int8)
    a = dev.DeviceArray.zeros(y.shape[0], np.float32)
    dev.residual_layer_norm(dev.DeviceArray.from_host(y), dev.DeviceArray.from_host(r),
                            dev.DeviceArray.from_host(g), dev.DeviceArray.from_host(b), out, q, a)
    dev.synchronize()
    got = out.host()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))  # bit for bit, signed zeros too
    assert np.array_equal(q.host(), q_ref) and np.array_equal(a.host(), a_ref)
    # non-finite inputs: the same positions turn NaN / infinite, and the flag is set
    y2 = y[:4].copy()
    y2[0, 100] = np.nan
    y2[1, 300] = np.inf
    y2[2, 5] = -np.inf
    ref2 = orc.residual_layer_norm(y2, r[:4], g, b)
    out2 = dev.DeviceArray.zeros(y2.shape, np.float32)
    err = dev.DeviceArray.zeros(1, np.int32)
    dev.residual_layer_norm(dev.DeviceArray.from_host(y2), dev.DeviceArray.from_host(r[:4]),
                            dev.DeviceArray.from_host(g), dev.DeviceArray.from_host(b), out2, err=err)
    dev.synchronize()
    got2 = out2.host()
    assert np.array_equal(np.isnan(got2), np.isnan(ref2))
    fin = ~np.isnan(ref2)
    assert np.array_equal(got2[fin], ref2[fin])
    assert err.host()[0] == 1


def _attention_case(pkg, orc, dev, q, k, v, cu, heads, bf16):
    T = q.shape[0]
    lens = np.diff(cu.astype(np.int64))
    seq = np.repeat(np.arange(len(lens), dtype=np.int32), lens)
    if bf16:
        qh, kh, vh = (pkg.synthetic.bf16_round(x) for x in (q, k, v))
        q, k, v = (pkg.synthetic.bf16_to_f32(x) for x in (qh, kh, vh))
        dq, dk, dv = (dev.DeviceArray.from_host(x) for x in (qh, kh, vh))
    else:
        dq, dk, dv = (dev.DeviceArray.from_host(x) for x in (q, k, v))
    ref = orc.attention(q, k, v, cu, cu, heads)
    dseq, dcu = dev.DeviceArray.from_host(seq), dev.DeviceArray.from_host(cu)
    # packed_self: the key-staging kernel (ranges up to 256 keys); otherwise
    # one wave per (row, head).
    for packed in (True, False):
        out = dev.DeviceArray.zeros((T, heads * 64), np.float32)
        dev.attention(dq, dk, dv, dseq, dcu, out, heads=heads, max_keys=int(lens.max()), bf16=bf16,
                      packed_self=packed)
        dev.synchronize()
        got = out.host()
        assert rel_err(got, ref) <= REL_TOL or np.max(np.abs(got - ref)) < 1e-5
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
            f"attention not bit-identical (packed_self={packed})"


@pytest.mark.parametrize("bf16", [False, True])
def test_varlen_attention_full_workload(pkg, orc, dev, bf16):
    q, k, v, cu = pkg.attention_inputs()
    print(f"attention T={q.shape[0]} bf16={bf16}", flush=True)
    _attention_case(pkg, orc, dev, q, k, v, cu, 8, bf16)


@pytest.mark.parametrize("bf16", [False, True])
def test_cross_attention_decode_shape(pkg, orc, dev, bf16):
    """The 256-sentence attention workload as cross-attention: one query per
    sentence (cu_q != cu_k) over that sentence's packed keys and values."""
    q, k, v, cu = pkg.attention_inputs()
    B = len(cu) - 1
    lens = np.diff(cu.astype(np.int64))
    qc = np.ascontiguousarray(q[cu[:-1].astype(np.int64)])
    if bf16:
        qh, kh, vh = (pkg.synthetic.bf16_round(x) for x in (qc, k, v))
        qc, k, v = (pkg.synthetic.bf16_to_f32(x) for x in (qh, kh, vh))
        dq, dk, dv = (dev.DeviceArray.from_host(x) for x in (qh, kh, vh))
    else:
        dq, dk, dv = (dev.DeviceArray.from_host(x) for x in (qc, k, v))
    cu_q = np.arange(B + 1, dtype=np.uint32)
    ref = orc.attention(qc, k, v, cu_q, cu, 8)
    print(f"cross-attention B={B} T={k.shape[0]} bf16={bf16}", flush=True)
    out = dev.DeviceArray.zeros((B, 512), np.float32)
    dev.attention(dq, dk, dv, dev.DeviceArray.from_host(np.arange(B, dtype=np.int32)),
                  dev.DeviceArray.from_host(cu), out, heads=8, max_keys=int(lens.max()), bf16=bf16,
                  packed_self=False)
    dev.synchronize()
    got = out.host()
    assert rel_err(got, ref) <= REL_TOL
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "cross-attention not bit-identical"


def test_attention_edges(pkg, orc, dev):
    rng = np.random.default_rng(14)
    # single key, 64/65 keys (chunk boundary), a 1000-key row (large variant),
    # and the reference's masking KAT shape at head_dim 64
    lens = np.array([1, 64, 65, 2, 1000, 3], np.int64)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    T = int(cu[-1])
    q, k, v = (rng.standard_normal((T, 128)).astype(np.float32) for _ in range(3))
    print("attention edges", flush=True)
    _attention_case(pkg, orc, dev, q, k, v, cu, 2, False)
    # ranges of 1..256 keys around the staging kernel's batch and chunk edges
    lens = np.array([1, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 2],
                    np.int64)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    T = int(cu[-1])
    q, k, v = (rng.standard_normal((T, 512)).astype(np.float32) for _ in range(3))
    print("attention edges up to 256 keys", flush=True)
    _attention_case(pkg, orc, dev, q, k, v, cu, 8, False)


@pytest.mark.parametrize("M", [1, 64, 130])
def test_vocab_argmax_matches_oracle(pkg, orc, dev, full_model, M):
    """Up to 64 rows one row group; 130 rows run three 64-row groups side
    by side, the last one holding two rows."""
    m = full_model
    rng = np.random.default_rng(15 + M)
    x = rng.standard_normal((M, 512)).astype(np.float32)
    q_ref, a_ref = orc.quantize_rows(x)
    logits_ref, _, _, _ = orc.linear_forward(x, m.embedding, m.embedding_mult, m.output_bias)
    masked = np.zeros(m.geometry.vocab, bool)
    masked[1] = True
    masked[7:39] = True
    lm = np.where(masked[None, :], -np.inf, logits_ref).astype(np.float32)
    tok_ref = np.argmax(lm, axis=1)  # first maximum = lowest id
    dq, da = dev.DeviceArray.from_host(q_ref), dev.DeviceArray.from_host(a_ref)
    demb, dmult, dbias = (dev.DeviceArray.from_host(t) for t in
                          (m.embedding, m.embedding_mult, m.output_bias))
    tok = dev.DeviceArray.zeros(M, np.int32)
    logits = dev.DeviceArray.zeros((M, m.geometry.vocab), np.float32)
    dev.vocab_argmax(dq, da, demb, dmult, dbias, tok, logits)
    dev.synchronize()
    assert np.array_equal(tok.host(), tok_ref)
    got = logits.host()
    assert np.array_equal(got, lm)


def test_vocab_argmax_ties_pick_lowest_id(pkg, dev):
    V, K = 4096, 64
    emb = np.zeros((V, K), np.int8)
    emb[:, 0] = 1
    emb[[5, 700, 3000, 4095], 0] = 9  # four equal maxima
    mult = np.ones(V, np.float32)
    bias = np.zeros(V, np.float32)
    xq = np.zeros((3, K), np.int8)
    xq[:, 0] = 127
    xa = np.ones(3, np.float32)
    tok = dev.DeviceArray.zeros(3, np.int32)
    args = [dev.DeviceArray.from_host(t) for t in (xq, xa, emb, mult, bias)]
    dev.vocab_argmax(*args, tok)
    dev.synchronize()
    assert tok.host().tolist() == [5, 5, 5]
    emb[5, 0] = 1
    emb[700, 0] = 1
    args = [dev.DeviceArray.from_host(t) for t in (xq, xa, emb, mult, bias)]
    dev.vocab_argmax(*args, tok)
    dev.synchronize()
    assert tok.host().tolist() == [3000, 3000, 3000]
    # a masked id never wins (id 20 is in 7..38) unless the mask is off
    emb[20, 0] = 100
    args = [dev.DeviceArray.from_host(t) for t in (xq, xa, emb, mult, bias)]
    dev.vocab_argmax(*args, tok)
    dev.synchronize()
    assert tok.host().tolist() == [3000, 3000, 3000]
    dev.vocab_argmax(*args, tok, flags=pkg.FLAG_NO_GENERATION_MASK)
    dev.synchronize()
    assert tok.host().tolist() == [20, 20, 20]


@pytest.mark.gpu
def test_vocab_argmax_nonfinite_logits_follow_strict_scan(pkg, dev):
    """The reference scores with a strict '>' scan from -inf that starts at the
    first unmasked id (q8_engine.rs:749-790): NaN never wins, a row whose
    logits are all -inf or NaN yields its first candidate, and -0.0 ties with
    +0.0.  Zero activations make every logit equal to its bias."""
    V, K = 4096, 64
    emb = np.zeros((V, K), np.int8)
    mult = np.ones(V, np.float32)
    xq = np.zeros((2, K), np.int8)
    xa = np.ones(2, np.float32)

    def run(bias):
        tok = dev.DeviceArray.zeros(2, np.int32)
        args = [dev.DeviceArray.from_host(t) for t in (xq, xa, emb, mult, bias)]
        dev.vocab_argmax(*args, tok)
        dev.synchronize()
        return tok.host().tolist()

    b = np.full(V, -np.inf, np.float32)
    b[[0, 2, 900]] = np.nan
    assert run(b) == [0, 0]          # only -inf / NaN: first candidate (id 0)
    b[0] = -np.inf
    b[[3, 4]] = np.nan
    assert run(b) == [0, 0]
    b[3000] = -5.0
    b[3001] = np.nan
    assert run(b) == [3000, 3000]    # the one finite logit wins over NaN
    b = np.full(V, -1.0, np.float32)
    b[50] = -0.0
    b[100] = 0.0
    assert run(b) == [50, 50]        # -0.0 == +0.0: the lower id
    b[50] = 0.0
    b[100] = -0.0
    assert run(b) == [50, 50]


# ---- static activation multiplier (the reference's Q8 models) ---------------------
@pytest.mark.parametrize("K,N", [(512, 1536), (2048, 512), (512, 32000)])
@pytest.mark.parametrize("M", [1, 8, 64, 256])
def test_q8_linear_static_matches_oracle(pkg, orc, dev, M, K, N):
    a, w, mult, bias = pkg.gemm_inputs(M, K, N, seed=9)
    act = float(np.float32(127) / np.float32(np.abs(a).max() * 0.75))  # a few saturate
    print(f"q8_linear_static M={M} K={K} N={N} act_mult={act:.4f}", flush=True)
    y_ref, acc_ref, _ = orc.linear_forward_static(a, w, mult, bias, act, threads=16)
    da, dw, dm, db = (dev.DeviceArray.from_host(x) for x in (a, w, mult, bias))
    di = dev.DeviceArray.zeros((M, N), np.int32)
    df = dev.DeviceArray.zeros((M, N), np.float32)
    err = dev.DeviceArray.zeros(1, np.int32)
    dev.q8_linear_static(da, act, dw, dm, db, di, df, err=err)
    dev.synchronize()
    assert err.host()[0] == 0
    assert np.array_equal(di.host(), acc_ref), "i32 accumulators differ"
    assert np.array_equal(df.host().view(np.uint32), y_ref.view(np.uint32))


def test_q8_linear_static_reference_kat(pkg, dev, kats):
    """q8_gemm.rs:620-668 on the GPU: K padded to 64 with zero activations
    and weights (quantized to 0, so the accumulators are unchanged)."""
    k = kats["linear_integer_oracle"]
    w = np.zeros((2, 64), np.int8)
    w[:, :4] = np.array(k["weights_out_in"], np.int8)
    mult = np.full(2, k["weight_mult"], np.float32)
    bias = np.array(k["bias"], np.float32)
    dw, dm, db = (dev.DeviceArray.from_host(x) for x in (w, mult, bias))
    for rows in k["inputs"]:
        x = np.zeros((len(rows), 64), np.float32)
        x[:, :4] = np.array(rows, np.float32)
        q = np.clip(np.rint(x * 4.0), -127, 127).astype(np.int64)
        expected = (q @ w.T.astype(np.int64)).astype(np.float32) / np.float32(32.0) + bias
        dx = dev.DeviceArray.from_host(x)
        df = dev.DeviceArray.zeros((len(rows), 2), np.float32)
        dev.q8_linear_static(dx, k["activation_mult"], dw, dm, db, None, df)
        dev.synchronize()
        assert np.array_equal(df.host(), expected)


@pytest.mark.parametrize("d", [64, 384, 512])
@pytest.mark.parametrize("rows", [1, 7, 300])
def test_ssru_layer_norm_matches_oracle(pkg, orc, dev, rows, d):
    rng = np.random.default_rng(rows * 1000 + d)
    c, f, s, r = (rng.standard_normal((rows, d)).astype(np.float32) * 2 for _ in range(4))
    f[0, :8] = [np.inf, -np.inf, 0.0, -0.0, 88.7, -88.7, 104.0, -104.0]  # gate saturation edges
    s[0, 8:12] = [-0.0, 0.0, -1e-30, 1e-30]
    g = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    b = (0.1 * rng.standard_normal(d)).astype(np.float32)
    out_ref, st_ref = orc.ssru_layer_norm(c, f, s, r, g, b)
    q_ref, a_ref = orc.quantize_rows(out_ref)
    print(f"ssru rows={rows} d={d}", flush=True)
    dc, dfg, ds, dr, dg, dbb = (dev.DeviceArray.from_host(x) for x in (c, f, s, r, g, b))
    out = dev.DeviceArray.zeros((rows, d), np.float32)
    q = dev.DeviceArray.zeros((rows, d), np.int8)
    a = dev.DeviceArray.zeros(rows, np.float32)
    err = dev.DeviceArray.zeros(1, np.int32)
    dev.ssru_layer_norm(dc, dfg, ds, dr, dg, dbb, out, q=q, a=a, err=err)
    dev.synchronize()
    assert err.host()[0] == 0
    assert np.array_equal(ds.host().view(np.uint32), st_ref.view(np.uint32)), "state differs"
    assert np.array_equal(out.host().view(np.uint32), out_ref.view(np.uint32)), "output differs"
    assert np.array_equal(q.host(), q_ref) and np.array_equal(a.host(), a_ref)


# ---- lexical shortlist: scoring only the candidate ids ----------------------------
def test_candidate_argmax_matches_oracle(pkg, orc, dev, full_model):
    import importlib

    sl = importlib.import_module(pkg.__name__ + ".shortlist")
    m = full_model
    V, K = m.geometry.vocab, m.geometry.dim
    rng = np.random.default_rng(33)
    # a synthetic shortlist: 100 source ids, 40 targets each, firstNum 100
    src_v = 100
    offs_t = np.arange(0, 40 * src_v + 1, 40, dtype=np.int64)
    targets = rng.integers(0, V, size=40 * src_v).astype(np.uint32)
    short = sl.LexicalShortlist.from_bytes(sl.LexicalShortlist.to_bytes(100, offs_t, targets), src_v, V)
    lists = [short.candidates(rng.integers(0, src_v, size=n)) for n in (3, 17, 60, 1)]
    lists.append(sl.LexicalShortlist.from_bytes(None, src_v, V).candidates([]))  # the full vocabulary
    M = len(lists)
    xq = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
    xa = rng.uniform(1.0, 50.0, size=M).astype(np.float32)
    flat, offs, mx = sl.pack_candidates(lists)
    tok_ref, lg_ref = orc.candidate_argmax(xq, xa, m.embedding, m.embedding_mult, m.output_bias,
                                           flat, offs)
    print(f"candidate_argmax: {M} rows, list lengths {np.diff(offs).tolist()}", flush=True)
    d = {k: dev.DeviceArray.from_host(v) for k, v in dict(
        xq=xq, xa=xa, emb=m.embedding, mult=m.embedding_mult, bias=m.output_bias, cand=flat,
        offs=offs).items()}
    tok = dev.DeviceArray.zeros(M, np.int32)
    lg = dev.DeviceArray.zeros(flat.size, np.float32)
    err = dev.DeviceArray.zeros(1, np.int32)
    dev.candidate_argmax(d["xq"], d["xa"], d["emb"], d["mult"], d["bias"], d["cand"], d["offs"], mx,
                         tok, logits=lg, err=err)
    dev.synchronize()
    assert err.host()[0] == 0
    assert np.array_equal(tok.host(), tok_ref)
    assert np.array_equal(lg.host().view(np.uint32), lg_ref.view(np.uint32))
    # the full-vocabulary list scores like the vocabulary kernel (masked ids excluded)
    dt = dev.DeviceArray.zeros(1, np.int32)
    dev.vocab_argmax(dev.DeviceArray.from_host(xq[-1:]), dev.DeviceArray.from_host(xa[-1:]),
                     d["emb"], d["mult"], d["bias"], dt)
    dev.synchronize()
    assert dt.host()[0] == tok.host()[-1]


def test_candidate_argmax_ties_and_bad_ids(pkg, orc, dev):
    rng = np.random.default_rng(35)
    V, K = 300, 64
    emb = rng.integers(-127, 128, size=(V, K)).astype(np.int8)
    emb[201] = emb[200]
    mult = np.full(V, 100.0, np.float32)
    bias = np.zeros(V, np.float32)
    xq = emb[200:201].copy()
    xa = np.ones(1, np.float32)
    cand = np.array([0, 5, 200, 201, 250], np.uint32)
    offs = np.array([0, 5], np.uint32)
    tok_ref, _ = orc.candidate_argmax(xq, xa, emb, mult, bias, cand, offs)
    assert tok_ref[0] == 200
    D = dev.DeviceArray.from_host
    tok = dev.DeviceArray.zeros(1, np.int32)
    err = dev.DeviceArray.zeros(1, np.int32)
    dev.candidate_argmax(D(xq), D(xa), D(emb), D(mult), D(bias), D(cand), D(offs), 5, tok, err=err)
    dev.synchronize()
    assert tok.host()[0] == 200 and err.host()[0] == 0
    bad = np.array([0, 5, 200, V + 7, 201], np.uint32)
    dev.candidate_argmax(D(xq), D(xa), D(emb), D(mult), D(bias), D(bad), D(offs), 5, tok, err=err)
    dev.synchronize()
    assert err.host()[0] == 1 and tok.host()[0] == 200


@pytest.mark.parametrize("packed", [True, False])
def test_attention_head_dim_48(pkg, orc, dev, packed):
    """Heads of width 48 (the reference's 384-wide, 8-head model): packed
    self-attention (key-staging kernel, ranges up to 256 keys) and the
    one-wave-per-(row, head) kernel, against the oracle bit for bit."""
    rng = np.random.default_rng(48)
    lens = np.array([1, 5, 47, 64, 65, 130, 256, 3], np.int64)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    T = int(cu[-1])
    q, k, v = (rng.standard_normal((T, 384)).astype(np.float32) for _ in range(3))
    ref = orc.attention(q, k, v, cu, cu, 8)
    seq = np.repeat(np.arange(len(lens), dtype=np.int32), lens)
    D = dev.DeviceArray.from_host
    out = dev.DeviceArray.zeros((T, 384), np.float32)
    dev.attention(D(q), D(k), D(v), D(seq), D(cu), out, heads=8, max_keys=int(lens.max()),
                  packed_self=packed, head_dim=48)
    dev.synchronize()
    assert np.array_equal(out.host().view(np.uint32), ref.view(np.uint32))
    # cross-attention shape: one query per sequence
    B = len(lens)
    qc = np.ascontiguousarray(q[cu[:-1].astype(np.int64)])
    refc = orc.attention(qc, k, v, np.arange(B + 1, dtype=np.uint32), cu, 8)
    outc = dev.DeviceArray.zeros((B, 384), np.float32)
    dev.attention(D(qc), D(k), D(v), D(np.arange(B, dtype=np.int32)), D(cu), outc, heads=8,
                  max_keys=int(lens.max()), packed_self=False, head_dim=48)
    dev.synchronize()
    assert np.array_equal(outc.host().view(np.uint32), refc.view(np.uint32))
