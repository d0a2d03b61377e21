"""The llama2c decoder on the GPU: each kernel through the C ABI against the
decoder oracle, whole decodes through the C ABI, and the application under the
loom_private protocol (the cases of
applications/loom_private/decoder/tests/run_tests.sh:37-75)."""
import numpy as np
import pytest

import decoder_oracle as dorc

pytestmark = pytest.mark.gpu


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("width,vocab", [(96, 16), (2, 2), (4100, 300), (1001, 77)])
def test_init_model_exact(torch_gpu, l2c, width, vocab):
    torch = torch_gpu
    print(f"case init_model width={width} vocab={vocab}", flush=True)
    emb = torch.empty(vocab * width, dtype=torch.float32, device="cuda")
    cls = torch.empty(vocab * width, dtype=torch.float32, device="cuda")
    w = torch.empty(width, dtype=torch.float32, device="cuda")
    l2c.decoder_init_model(emb, cls, w, width, vocab)
    torch.cuda.synchronize()
    e, c, g = dorc.model(width, vocab)
    np.testing.assert_array_equal(emb.cpu().numpy().reshape(vocab, width), e)
    np.testing.assert_array_equal(cls.cpu().numpy().reshape(vocab, width), c)
    np.testing.assert_array_equal(w.cpu().numpy(), g)


@pytest.mark.parametrize("width,vocab,batch", [(96, 16, 40), (4100, 300, 9), (1001, 77, 30), (2, 2, 3),
                                               (16384, 40, 7), (16384, 40, 513), (12000, 33, 520),
                                               (16384, 64, 1024)])
def test_rmsnorm_synthetic_exact(torch_gpu, l2c, width, vocab, batch):
    """The contract's float32 order on the synthetic model, bit for bit; an
    invalid token gives a NaN row."""
    torch = torch_gpu
    print(f"case decoder_rmsnorm width={width} vocab={vocab} batch={batch}", flush=True)
    e, _, w = dorc.model(width, vocab)
    tokens = (np.arange(batch) * 7 % vocab).astype(np.int32)
    tokens[batch // 2] = -1
    tokens[-1] = vocab
    out = torch.empty(batch * width, dtype=torch.float32, device="cuda")
    l2c.decoder_rmsnorm(out, dev(torch, tokens), dev(torch, e), dev(torch, w), width, vocab, batch)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(batch, width)
    for b in range(batch):
        if 0 <= tokens[b] < vocab:
            np.testing.assert_array_equal(got[b], dorc.rmsnorm_f32(e[tokens[b]][None], w)[0])
        else:
            assert np.isnan(got[b]).all()


@pytest.mark.parametrize("width,vocab,batch", [(3000, 50, 64), (16384, 50, 65), (16384, 50, 601)])
def test_rmsnorm_general_rows(torch_gpu, l2c, width, vocab, batch):
    """Arbitrary embedding rows: within 2e-6 relative of the double result."""
    torch = torch_gpu
    print(f"case decoder_rmsnorm general width={width} batch={batch}", flush=True)
    rng = np.random.default_rng(11)
    e = rng.standard_normal((vocab, width)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, width).astype(np.float32)
    tokens = rng.integers(0, vocab, batch).astype(np.int32)
    out = torch.empty(batch * width, dtype=torch.float32, device="cuda")
    l2c.decoder_rmsnorm(out, dev(torch, tokens), dev(torch, e), dev(torch, w), width, vocab, batch)
    torch.cuda.synchronize()
    x = e[tokens].astype(np.float64)
    ref = w * (x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + 1e-5))
    assert dorc.within(out.cpu().numpy().reshape(batch, width), ref, 2e-6).all()


@pytest.mark.parametrize("vocab,batch", [(8192, 33), (1000, 17), (77, 5), (2, 4), (8192, 513), (6000, 520)])
def test_softmax_argmax(torch_gpu, l2c, vocab, batch):
    torch = torch_gpu
    print(f"case decoder_softmax_argmax vocab={vocab} batch={batch}", flush=True)
    rng = np.random.default_rng(vocab)
    logits = (rng.standard_normal((batch, vocab)) * 3).astype(np.float32)
    logits[0, :] = 0.5  # all equal: the first maximum is index 0
    logits[batch - 2, :] = 0.25  # again in a later row (the second of a two-row workgroup)
    steps, step = 3, 1
    probs = torch.empty(batch * vocab, dtype=torch.float32, device="cuda")
    tokens = torch.full((batch,), -5, dtype=torch.int32, device="cuda")
    generated = torch.full((batch * steps,), -7, dtype=torch.int32, device="cuda")
    l2c.decoder_softmax_argmax(probs, dev(torch, logits), tokens, generated, vocab, batch, steps, step)
    torch.cuda.synchronize()
    p = probs.cpu().numpy().reshape(batch, vocab)
    l64 = logits.astype(np.float64)
    ref = np.exp(l64 - l64.max(axis=1, keepdims=True))
    ref /= ref.sum(axis=1, keepdims=True)
    assert dorc.within(p, ref, dorc.PROBABILITY_RELATIVE).all()
    want = np.argmax(p, axis=1)  # first maximum of the float32 probabilities
    assert np.array_equal(tokens.cpu().numpy(), want)
    assert want[0] == 0 and want[batch - 2] == 0
    g = generated.cpu().numpy().reshape(batch, steps)
    assert np.array_equal(g[:, step], want)
    assert (g[:, 0] == -7).all() and (g[:, 2] == -7).all()


@pytest.mark.parametrize("vocab,batch,nan_rows", [(64, 2, [1]), (8192, 600, [1, 300, 599])])
def test_softmax_argmax_nan_row(torch_gpu, l2c, vocab, batch, nan_rows):
    """A row of NaN logits has no maximum: token -1 (first and second row of a
    two-row workgroup alike)."""
    torch = torch_gpu
    print(f"case decoder_softmax_argmax nan rows vocab={vocab} batch={batch}", flush=True)
    logits = np.zeros((batch, vocab), np.float32)
    logits[nan_rows] = np.nan
    probs = torch.empty(batch * vocab, dtype=torch.float32, device="cuda")
    tokens = torch.zeros(batch, dtype=torch.int32, device="cuda")
    generated = torch.zeros(batch * 2, dtype=torch.int32, device="cuda")
    l2c.decoder_softmax_argmax(probs, dev(torch, logits), tokens, generated, vocab, batch, 2, 0)
    torch.cuda.synchronize()
    want = np.zeros(batch, np.int32)
    want[nan_rows] = -1
    assert tokens.cpu().numpy().tolist() == want.tolist()


@pytest.mark.parametrize("batch,width,vocab,steps", [(40, 96, 16, 5), (70, 200, 33, 4), (3, 2, 2, 2),
                                                     (300, 1000, 250, 3)])
def test_decode_through_abi(torch_gpu, l2c, batch, width, vocab, steps):
    """A whole decode through the C ABI (init, then per step rmsnorm ->
    l2c_matmul -> softmax_argmax with on-device feedback), every sequence
    against the dense double oracle."""
    torch = torch_gpu
    print(f"case decode batch={batch} width={width} vocab={vocab} steps={steps}", flush=True)
    f32 = torch.float32
    emb = torch.empty(vocab * width, dtype=f32, device="cuda")
    cls = torch.empty(vocab * width, dtype=f32, device="cuda")
    w = torch.empty(width, dtype=f32, device="cuda")
    l2c.decoder_init_model(emb, cls, w, width, vocab)
    tokens = dev(torch, dorc.prompts(batch, vocab))
    generated = torch.full((batch * steps,), -1, dtype=torch.int32, device="cuda")
    norm = torch.empty((steps, batch, width), dtype=f32, device="cuda")
    logits = torch.empty((steps, batch, vocab), dtype=f32, device="cuda")
    probs = torch.empty((steps, batch, vocab), dtype=f32, device="cuda")
    for s in range(steps):
        l2c.decoder_rmsnorm(norm[s], tokens, emb, w, width, vocab, batch)
        l2c.matmul(logits[s], norm[s], cls, batch, width, vocab)
        l2c.decoder_softmax_argmax(probs[s], logits[s], tokens, generated, vocab, batch, steps, s)
    torch.cuda.synchronize()
    gen = generated.cpu().numpy().reshape(batch, steps)
    assert np.array_equal(gen, dorc.analytic_tokens(batch, vocab, steps))
    o, l, p = norm.cpu().numpy(), logits.cpu().numpy(), probs.cpu().numpy()
    sq_ok, sum_ok = dorc.invariants(o, p, width, vocab)
    assert sq_ok.all() and sum_ok.all()
    for b in range(batch):
        eo, el, ep, _ = dorc.dense_double(b % vocab, width, vocab, steps)
        assert dorc.within(o[:, b], eo, dorc.NORMALIZED_RELATIVE).all()
        assert dorc.within(l[:, b], el, dorc.LOGIT_RELATIVE).all()
        assert dorc.within(p[:, b], ep, dorc.PROBABILITY_RELATIVE).all()


def decoder(l2c, args):
    code, record, err = l2c.decoder(args, timeout=300)
    print(err[-2000:], flush=True)
    return code, record, err


def sets(batch, width, vocab, steps, *extra):
    out = ["--set", f"batch={batch}", "--set", f"width={width}", "--set", f"vocab={vocab}", "--set",
           f"steps={steps}"]
    for e in extra:
        out += ["--set", e]
    return out


@pytest.mark.parametrize("name,args,needle", [
    ("wraparound", sets(40, 96, 16, 5), "PASS: 0/200 tokens wrong"),
    ("minimum", sets(3, 2, 2, 2), "PASS"),
    ("square", sets(1030, 1000, 1000, 3), "PASS"),
    ("wide", sets(1, 4100, 300, 2), "PASS"),
    ("graph-only", ["--launch", "graph"] + sets(70, 200, 33, 4), "graph invocation 2: PASS"),
])
def test_application_check_cases(torch_gpu, l2c, name, args, needle):
    print(f"case decoder check {name}", flush=True)
    code, record, err = decoder(l2c, args)
    assert code == 0, err
    assert needle in err
    assert record["status"] == "pass" and record["outputs_agree"] is True
    assert record["identity"] == "loom-private/llama2c-decoder"
    digests = {c["digest"] for c in record["checks"]}
    assert len(digests) == 1 and all(c["pass"] for c in record["checks"])
    assert len(record["checks"]) == (2 if name == "graph-only" else 4)


@pytest.mark.parametrize("fault,needle", [
    (1, "token mismatch sequence 39 step 4: expected 12, actual 13"),
    (2, "invariant failure sequence 20 step 4"),
    (3, "probability mismatch sequence 0 step 4 index 8: expected"),
])
def test_application_detects_planted_faults(torch_gpu, l2c, fault, needle):
    print(f"case decoder fault={fault}", flush=True)
    code, record, err = decoder(l2c, sets(40, 96, 16, 5, f"fault={fault}"))
    assert code == 1
    assert needle in err
    assert record["status"] == "fail"


def test_application_large_check(torch_gpu, l2c):
    """The contract's large shape (1024 sequences, width 16384, vocab 8192,
    4 steps), direct and graph, two invocations each."""
    print("case decoder large check", flush=True)
    code, record, err = decoder(l2c, [])
    assert code == 0, err
    assert "PASS: 0/4096 tokens wrong" in err
    assert record["dimensions"]["classifier_macs_per_step"] == 1024 * 8192 * 16384


def test_application_bench_and_in_process(torch_gpu, l2c):
    print("case decoder bench graph", flush=True)
    code, record, err = decoder(l2c, ["--action", "bench", "--launch", "graph", "--iterations", "3",
                                      "--warmup", "1"])
    assert code == 0, err
    assert record["status"] == "unvalidated_bench"
    t = record["timing"]["compute"]
    assert t["batch_per_iteration_us"] > 0 and len(t["single_us"]) == 3
    print("case decoder in-process check", flush=True)
    code, record, _ = l2c.decoder(sets(40, 96, 16, 5), in_process=True)
    assert code == 0 and record["status"] == "pass"


@pytest.mark.parametrize("width,vocab,batch", [(16384, 50, 1024), (16384, 60, 601), (16384, 50, 65), (3000, 50, 64),
                                               (1001, 40, 7), (20000, 30, 3)])
def test_rmsnorm_absmax(torch_gpu, l2c, width, vocab, batch):
    """l2c_decoder_rmsnorm_absmax writes what l2c_decoder_rmsnorm writes, bit for
    bit, and raises the word to max |normalized| over the batch (NaN rows of
    out-of-range tokens ignored). Shapes cover the two-row pipelined kernel
    (16384 wide, batch >= 512, with a ragged last pair at 601), the
    register-resident kernels (aligned and not: width 1001) and the streamed
    one (20000).
    A second call from a word already above the batch's maximum leaves it
    there."""
    torch = torch_gpu
    print(f"case decoder_rmsnorm_absmax width={width} vocab={vocab} batch={batch}", flush=True)
    rng = np.random.default_rng(width + batch)
    e = (rng.standard_normal((vocab, width)) * 3.0).astype(np.float32)
    w = rng.uniform(-1.5, 1.5, width).astype(np.float32)
    tokens = rng.integers(0, vocab, batch).astype(np.int32)
    tokens[::5] = vocab + 3  # out of range: NaN rows
    tokens[1] = 0
    td, ed, wd = dev(torch, tokens), dev(torch, e), dev(torch, w)
    plain = torch.empty(batch * width, dtype=torch.float32, device="cuda")
    fused = torch.full((batch * width,), 7.0, dtype=torch.float32, device="cuda")
    word = torch.zeros(1, dtype=torch.int32, device="cuda")
    l2c.decoder_rmsnorm(plain, td, ed, wd, width, vocab, batch)
    l2c.decoder_rmsnorm_absmax(fused, td, ed, wd, width, vocab, batch, word)
    torch.cuda.synchronize()
    p, f = plain.cpu().numpy(), fused.cpu().numpy()
    np.testing.assert_array_equal(p.view(np.uint32), f.view(np.uint32))
    want = np.nanmax(np.abs(p))
    got = word.cpu().numpy().view(np.float32)[0]
    assert got == want, (got, want)
    high = np.float32(want * 2)
    word.copy_(torch.from_numpy(np.array([high], np.float32).view(np.int32)))
    l2c.decoder_rmsnorm_absmax(fused, td, ed, wd, width, vocab, batch, word)
    torch.cuda.synchronize()
    assert word.cpu().numpy().view(np.float32)[0] == high
