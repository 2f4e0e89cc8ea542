"""Device LM head (nls_lm_head) against the CPU restatement of nimllm's
`matmul` on the output matrix (oracle/nls_oracle_quant.c): logits bit-equal
for every weight type the reference reads, on both of its paths (int8
activations and dequantise + dotF32), with and without a LoRA adapter, and
at the Llama-3.2-1B output shape (128256 x 2048, Q6_K)."""
import numpy as np
import pytest

import oracle as O

F32 = np.float32
TYPES = O.GGML

# byte offsets of the fp16 scale fields inside one block, per type
HALF_FIELDS = {2: (0,), 3: (0, 2), 6: (0,), 7: (0, 2), 8: (0,), 10: (80, 82), 11: (108,),
               12: (0, 2), 13: (0, 2), 14: (208,)}


def rand_weights(t, rows, cols, rng):
    """Random GGUF rows of type t: every bit pattern is a valid block, except
    that the fp16 / fp32 scale fields are replaced by finite values of a
    modest size, as a quantiser writes them."""
    rb = O.row_bytes(t, cols)
    if t == 0:
        return rng.normal(size=(rows, cols)).astype(F32).view(np.uint8).reshape(rows, rb)
    if t in (1, 30):
        v = (rng.normal(size=(rows, cols)) * 0.5).astype(F32)
        if t == 1:
            return v.astype(np.float16).view(np.uint8).reshape(rows, rb)
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(rows, rb)
    raw = rng.integers(0, 256, size=(rows, rb), dtype=np.uint8)
    ts = O.type_size(t)
    blocks = raw.reshape(rows, rb // ts, ts)
    if t == 15:
        d = rng.uniform(1e-3, 2e-2, size=blocks.shape[:2]).astype(F32)
        blocks[:, :, 0:4] = d.view(np.uint8).reshape(blocks.shape[0], blocks.shape[1], 4)
    else:
        for off in HALF_FIELDS[t]:
            h = (rng.uniform(-1, 1, size=blocks.shape[:2]) * 2.0 ** rng.integers(-12, -4, size=blocks.shape[:2]))
            blocks[:, :, off:off + 2] = h.astype(np.float16).view(np.uint8).reshape(
                blocks.shape[0], blocks.shape[1], 2)
    return raw


def run_case(pkg, t, rows, cols, nb, exact=False, lora_rank=0, seed=0):
    import torch

    rng = np.random.default_rng(seed)
    w = rand_weights(t, rows, cols, rng)
    x = (rng.normal(size=(nb, cols)) * 2).astype(F32)
    lora = None
    lora_dev = None
    if lora_rank:
        a = (rng.normal(size=(lora_rank, cols)) * 0.05).astype(F32)
        b = (rng.normal(size=(rows, lora_rank)) * 0.05).astype(F32)
        lora = (a, b, 0.75)
        lora_dev = (torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), 0.75)
    want = O.matmul(t, w, rows, cols, x, exact=exact, lora=lora)
    y = pkg.lm_head(torch.from_numpy(w).cuda(), t, rows, cols, torch.from_numpy(x).cuda(), exact=exact,
                    lora=lora_dev)
    got = y.cpu().numpy()
    diff = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert diff.size == 0, (t, rows, cols, nb, exact, lora_rank, diff[:8], got.ravel()[diff[:4]],
                            want.ravel()[diff[:4]])


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["Q6_K", "Q4_K", "Q5_K", "Q8_0", "Q4_0"])
def test_int8_path_parity(pkg, name):
    t = TYPES[name]
    bs = O.block_size(t)
    cols_list = [256, 2048, 3072] if bs == 256 else [896, 2048, 2080]
    for ci, cols in enumerate(cols_list):
        for nb in (1, 2, 3, 4):
            print(f"lm_head int8 {name} rows=1000 cols={cols} nb={nb}", flush=True)
            run_case(pkg, t, 1000, cols, nb, seed=10 * ci + nb)
    # one hidden state over 3 or 4 passes of 2048 weights (rows streamed in a ring)
    big = 8192 if bs == 256 else 6144
    print(f"lm_head int8 {name} rows=300 cols={big} nb=1", flush=True)
    run_case(pkg, t, 300, big, 1, seed=77)
    if t != TYPES["Q8_0"]:  # Q8_0 takes the float path above 4 rows (model.nim:185)
        print(f"lm_head int8 {name} rows=333 cols={cols_list[1]} nb=9", flush=True)
        run_case(pkg, t, 333, cols_list[1], 9, seed=99)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(TYPES))
def test_float_path_parity(pkg, name):
    t = TYPES[name]
    bs = O.block_size(t)
    cols = 1000 if bs == 1 else (2080 if bs == 32 else 2048)
    for nb in (1, 5):
        print(f"lm_head float {name} rows=700 cols={cols} nb={nb}", flush=True)
        # exact=True forces the float path for the int8 types too
        run_case(pkg, t, 700, cols, nb, exact=True, seed=nb)
    if bs == 1:
        print(f"lm_head float {name} rows=257 cols=13 nb=2", flush=True)
        run_case(pkg, t, 257, 13, 2, seed=3)


@pytest.mark.gpu
def test_q8_0_batch_takes_float_path(pkg):
    # nb = 5 > 4: the reference dequantises Q8_0 rows instead (model.nim:185)
    assert not O.matmul_uses_act(8, 2048, 5)
    run_case(pkg, 8, 640, 2048, 5, seed=5)


@pytest.mark.gpu
@pytest.mark.parametrize("name,exact", [("Q6_K", False), ("Q4_K", True), ("F16", False)])
def test_lora_term_parity(pkg, name, exact):
    t = TYPES[name]
    print(f"lm_head lora {name} exact={exact}", flush=True)
    run_case(pkg, t, 500, 2048 if O.block_size(t) != 1 else 1024, 3, exact=exact, lora_rank=4, seed=21)


@pytest.mark.gpu
def test_llama_output_shape(pkg):
    """The Llama-3.2-1B output matrix (tied token embedding, Q6_K in the
    q4_k_m file): 128256 x 2048, one hidden state, every logit compared."""
    print("lm_head Q6_K 128256 x 2048 nb=1", flush=True)
    run_case(pkg, TYPES["Q6_K"], 128256, 2048, 1, seed=7)


@pytest.mark.gpu
def test_lm_head_feeds_sampler(pkg):
    """Logits written by nls_lm_head go straight into nls_sample: ids equal
    the oracle's sample of the oracle's logits."""
    import torch

    rng = np.random.default_rng(31)
    rows, cols, B = 32000, 2048, 4
    w = rand_weights(TYPES["Q6_K"], rows, cols, rng)
    x = (rng.normal(size=(B, cols)) * 2).astype(F32)
    want_logits = O.matmul(TYPES["Q6_K"], w, rows, cols, x)
    y = pkg.lm_head(torch.from_numpy(w).cuda(), TYPES["Q6_K"], rows, cols, torch.from_numpy(x).cuda())
    params = pkg.SamplerParams(temperature=0.8, topK=40, topP=0.95, minP=0.0, repeatPenalty=1.0,
                               repeatLastN=64, seed=5)
    s = pkg.BatchSampler([params] * B, rows)
    u = O.uniforms(5, B)
    ids = s.sample(y, u=torch.from_numpy(u).cuda()).cpu().numpy()
    s.close()
    p = O.make_params(temperature=0.8, topK=40, topP=0.95, minP=0.0, repeatPenalty=1.0, repeatLastN=64,
                      seed=5)
    want = [O.sample(p, want_logits[b], u=u[b], expf_mode=O.EXPF_CR)[0].id for b in range(B)]
    assert list(ids) == want


@pytest.mark.gpu
def test_lm_head_rejects_mismatched_tensors(pkg):
    """The wrapper refuses, before any launch, a weight of the wrong dtype or
    fewer than rows x rowBytes bytes, a cols that is not whole blocks, and
    LoRA tensors of the wrong shape."""
    import torch

    t, rows, cols = O.GGML["Q6_K"], 64, 512
    rb = int(pkg.lib().nls_lm_head_row_bytes(t, cols))
    assert rb == O.row_bytes(t, cols)
    assert pkg.lib().nls_lm_head_row_bytes(t, cols + 1) == -1
    assert pkg.lib().nls_lm_head_row_bytes(99, cols) == -1
    x = torch.zeros((1, cols), dtype=torch.float32, device="cuda")
    w = torch.zeros(rows * rb, dtype=torch.uint8, device="cuda")
    with pytest.raises(AssertionError):
        pkg.lm_head(w[:-1], t, rows, cols, x)
    with pytest.raises(AssertionError):
        pkg.lm_head(w.view(torch.int8), t, rows, cols, x)
    with pytest.raises(pkg.SamplerError):
        pkg.lm_head(w, t, rows, cols + 1, torch.zeros((1, cols + 1), dtype=torch.float32, device="cuda"))
    a = torch.zeros((4, cols), dtype=torch.float32, device="cuda")
    b = torch.zeros((rows, 4), dtype=torch.float32, device="cuda")
    with pytest.raises(AssertionError):
        pkg.lm_head(w, t, rows, cols, x, lora=(a, b[:, :3].contiguous(), 1.0))
    with pytest.raises(AssertionError):
        pkg.lm_head(w, t, rows, cols, x, lora=(a[:, :-1].contiguous(), b, 1.0))
    y = pkg.lm_head(w, t, rows, cols, x, lora=(a, b, 1.0))  # the well-formed call runs
    torch.cuda.synchronize()
    assert y.shape == (1, rows)


def _drawn_lm_case(i):
    """LM head sweep case i: (type, rows, cols, nb, exact, lora rank), drawn
    from a fixed seed with rows x cols x nb at most 40 M."""
    r = np.random.default_rng(500 + i)
    names = sorted(TYPES)
    while True:
        t = TYPES[names[int(r.integers(0, len(names)))]]
        bs = O.block_size(t)
        rows = int(r.choice([1, 7, 63, 64, 65, 300, 1000, 4099]))
        if bs == 1:
            cols = int(r.choice([1, 3, 17, 256, 1000, 2049, 4096]))
        elif bs == 32:
            cols = 32 * int(r.choice([1, 3, 8, 28, 65, 96, 192]))
        else:
            cols = 256 * int(r.choice([1, 2, 3, 8, 12, 16]))
        nb = int(r.choice([1, 2, 3, 4, 5, 8, 9, 16]))
        if rows * cols * nb <= 40_000_000:
            break
    return t, rows, cols, nb, bool(r.integers(0, 4) == 0), int(r.choice([0, 0, 1, 4, 16]))


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(24))
def test_lm_head_random_cases(pkg, i):
    """Twenty-four drawn cases over every weight type, row counts around the
    kernels' row groups (1, 63-65, 4099), column counts of one to many
    blocks, 1 to 16 hidden states (both of the reference's paths, model.nim:
    185), exactMatmul and LoRA ranks 0-16: every logit bit for bit."""
    t, rows, cols, nb, exact, rank = _drawn_lm_case(i)
    print(f"lm_head sweep {i}: type={t} rows={rows} cols={cols} nb={nb} exact={exact} lora={rank}", flush=True)
    run_case(pkg, t, rows, cols, nb, exact=exact, lora_rank=rank, seed=900 + i)
