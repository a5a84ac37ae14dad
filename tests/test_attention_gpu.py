"""GPU parity of the attention path (MI355X): q/k norm + RoPE + KV-cache write
(one launch) and the block attention over the static cache, against the
oracle on the same inputs and against the reference's own torch sequence.

Every attention form is covered: up to 32 query rows per KV head over at
most 4096 slots run as one launch -- one workgroup per KV head up to 256 (16
rows) or 384 (32 rows) valid slots, else several whose partials the last to
finish merges -- and the rest (the verify's 36 tokens x 4 query heads per KV
head among them) as chunked partials and a merge launch; a device-side valid
length below the host's bound trims either form's work.

qkv_rope_cache: q rows and every cache slot written equal the oracle within
one bf16 unit in the last place (the RMSNorm statistic may round either way;
more than 99% of values are bit-equal), and slots not addressed stay
untouched.  block_attention: within 2^-7 max|ref| + 1e-3 of the fp64 oracle
(the reference's bf16 bound) at the draft shape (4 rows, 16/8 heads) and the
verify shape (32 rows, 32/8 heads), ragged valid lengths, every GQA ratio, 256
query rows per KV head, masks with empty rows, fp16; bitwise deterministic;
graph replays equal eager calls.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt

pytestmark = pytest.mark.gpu
DEV = "cuda"
D = 128


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def rnd(*shape, dtype=torch.bfloat16, scale=1.0, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV, dtype=torch.float32) * scale).to(dtype)


def bound(ref):
    return 2 ** -7 * float(np.abs(ref).max()) + 1e-3


def fill_cache(cache, layer, L, seed, dtype=torch.bfloat16):
    k = rnd(cache.n_kv_heads, L, D, dtype=dtype, seed=seed)
    v = rnd(cache.n_kv_heads, L, D, dtype=dtype, seed=seed + 1)
    cache.store(layer, k, v)
    return k, v


@pytest.mark.parametrize("M,Hq,Hkv,L_valid,L_total", [(4, 16, 8, 1000, 1004), (32, 32, 8, 1024, 1056),
                                                      (8, 8, 8, 37, 64), (3, 12, 3, 301, 320),
                                                      (64, 32, 8, 530, 600), (1, 16, 8, 1, 32),
                                                      (8, 32, 8, 250, 288), (16, 16, 8, 256, 288),
                                                      (4, 16, 8, 2048, 2080), (4, 16, 8, 3001, 3040),
                                                      (8, 32, 8, 2600, 2624), (5, 10, 5, 63, 96),
                                                      (16, 16, 8, 1024, 1056), (2, 16, 8, 513, 544),
                                                      (16, 16, 8, 1800, 1856), (4, 16, 8, 4500, 4512),
                                                      (8, 32, 8, 4200, 4224), (9, 32, 8, 700, 736),
                                                      (16, 32, 8, 1000, 1024), (24, 32, 8, 3000, 3040),
                                                      (32, 32, 8, 64, 96), (32, 32, 8, 2000, 2048),
                                                      (33, 32, 8, 900, 928), (36, 32, 8, 1024, 1056),
                                                      (36, 32, 8, 300, 352), (12, 16, 8, 2500, 2528),
                                                      (36, 32, 8, 4200, 4224), (144, 32, 8, 600, 640)])
@pytest.mark.parametrize("masked", [False, True])
def test_block_attention_vs_oracle(M, Hq, Hkv, L_valid, L_total, masked):
    from kernels.attention_fused import BlockKVCache, block_attention
    print(f"block_attention M={M} Hq={Hq} Hkv={Hkv} L={L_valid} masked={masked}", flush=True)
    cache = BlockKVCache(1, Hkv, L_total - 32, 32, DEV)
    k, v = fill_cache(cache, 0, L_valid, seed=M + L_valid)
    q = rnd(M, Hq, D, seed=7)
    mask = None
    if masked:
        g = torch.Generator(device=DEV).manual_seed(11)
        mask = torch.rand(M, cache.full_len, generator=g, device=DEV) < 0.6
        mask[:, 0] = True
        if M > 2:
            mask[2] = False                       # a row with nothing visible -> zeros
    with torch.inference_mode():
        out = block_attention(q, cache, 0, mask=mask, valid_len=L_valid)
    torch.cuda.synchronize()
    ref = oatt.attention(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                         None if mask is None else mask[:, :L_valid].cpu().numpy(), D ** -0.5)
    got = out.view(M, Hq, D).float().cpu().numpy()
    err = float(np.abs(got - ref).max())
    assert err <= bound(ref), f"max err {err:.3e} > {bound(ref):.3e}"
    if masked and M > 2:
        assert np.all(got[2] == 0)


def test_block_attention_fp16_and_determinism():
    from kernels.attention_fused import BlockKVCache, block_attention
    cache = BlockKVCache(2, 8, 992, 32, DEV, dtype=torch.float16)
    k, v = fill_cache(cache, 1, 900, seed=3, dtype=torch.float16)
    q = rnd(16, 32, D, dtype=torch.float16, seed=4)
    with torch.inference_mode():
        a = block_attention(q, cache, 1, valid_len=900)
        b = block_attention(q, cache, 1, valid_len=900)
    assert torch.equal(a, b)
    ref = oatt.attention(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(), None, D ** -0.5)
    got = a.view(16, 32, D).float().cpu().numpy()
    assert float(np.abs(got - ref).max()) <= bound(ref)


@pytest.mark.parametrize("M,Hq,L_valid,L_total", [(4, 16, 900, 960), (32, 32, 1000, 1056),
                                                  (4, 16, 300, 352), (4, 16, 4500, 4544)])
def test_block_attention_ignores_nonfinite_slots_past_valid(M, Hq, L_valid, L_total):
    """Slots past the valid length that hold Inf/NaN (left by an earlier
    forward that overflowed) do not reach the output: every form (one
    workgroup per KV head, the split head form, the chunked form) matches the
    oracle over [0, L_valid) only, as the reference's SDPA does."""
    from kernels.attention_fused import BlockKVCache, block_attention
    print(f"nonfinite past valid M={M} Hq={Hq} L={L_valid}", flush=True)
    Hkv = 8
    cache = BlockKVCache(1, Hkv, L_total - 32, 32, DEV, dtype=torch.float16)
    k, v = fill_cache(cache, 0, L_valid, seed=41, dtype=torch.float16)
    n_bad = cache.full_len - L_valid
    bad = torch.full((Hkv, n_bad, D), float("inf"), device=DEV, dtype=torch.float16)
    bad[:, 1::2] = float("nan")
    cache.store(0, bad, bad, start=L_valid)
    q = rnd(M, Hq, D, dtype=torch.float16, seed=42)
    with torch.inference_mode():
        out = block_attention(q, cache, 0, valid_len=L_valid)
    torch.cuda.synchronize()
    got = out.view(M, Hq, D).float().cpu().numpy()
    assert np.isfinite(got).all()
    ref = oatt.attention(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(), None, D ** -0.5)
    assert float(np.abs(got - ref).max()) <= bound(ref)


def test_block_attention_matches_torch_sdpa_on_expanded_cache():
    """The reference's SDPA on its GQA-expanded [H_q, L, D] cache with the bool
    mask (adapters/base.py:245-262), computed in fp32 on the device."""
    from kernels.attention_fused import BlockKVCache, block_attention
    M, Hq, Hkv, L = 32, 32, 8, 700
    cache = BlockKVCache(1, Hkv, 736, 32, DEV)
    k, v = fill_cache(cache, 0, L, seed=21)
    q = rnd(M, Hq, D, seed=22)
    g = torch.Generator(device=DEV).manual_seed(5)
    mask = torch.rand(M, L, generator=g, device=DEV) < 0.8
    mask[:, :8] = True
    kk = k.float().repeat_interleave(Hq // Hkv, dim=0)[None]
    vv = v.float().repeat_interleave(Hq // Hkv, dim=0)[None]
    ref = F.scaled_dot_product_attention(q.float().transpose(0, 1)[None], kk, vv, attn_mask=mask[None, None],
                                         scale=D ** -0.5)[0].transpose(0, 1)
    with torch.inference_mode():
        out = block_attention(q, cache, 0, mask=mask, valid_len=L).view(M, Hq, D)
    err = float((out.float() - ref).abs().max())
    assert err <= 2 ** -7 * float(ref.abs().max()) + 1e-3


def _qkv_case(M, Hq, Hkv, n_pos, seed, dtype=torch.bfloat16):
    from kernels.attention_fused import default_inv_freq, rope_tables
    qkv = rnd(M, (Hq + 2 * Hkv) * D, dtype=dtype, scale=2.0, seed=seed)
    qn = (1 + 0.1 * rnd(D, dtype=torch.float32, seed=seed + 1)).to(dtype)
    kn = (1 + 0.1 * rnd(D, dtype=torch.float32, seed=seed + 2)).to(dtype)
    cos, sin = rope_tables(default_inv_freq(device=DEV), n_pos, dtype)
    return qkv, qn, kn, cos, sin


def _oracle_qkv(qkv, Hq, Hkv, qn, kn, cos, sin, pos, dtype="bf16"):
    M = qkv.shape[0]
    x = qkv.float().cpu().numpy().reshape(M, Hq + 2 * Hkv, D)
    c = cos.float().cpu().numpy()[pos.cpu().numpy()]
    s = sin.float().cpu().numpy()[pos.cpu().numpy()]
    q = oatt.qk_norm_rope(x[:, :Hq], None if qn is None else qn.float().cpu().numpy(), 1e-6, c, s, dtype)
    k = oatt.qk_norm_rope(x[:, Hq:Hq + Hkv], None if kn is None else kn.float().cpu().numpy(), 1e-6, c, s, dtype)
    return q, k, x[:, Hq + Hkv:]


def _close_ulp(got, ref, dtype="bf16"):
    ulp = 2.0 ** (-7 if dtype == "bf16" else -10)
    assert np.all(np.abs(got - ref) <= ulp * np.abs(ref) + 1e-30)
    assert (got != ref).mean() < 0.01


@pytest.mark.parametrize("M,Hq,Hkv", [(4, 16, 8), (32, 32, 8), (7, 8, 8), (8, 12, 4)])
@pytest.mark.parametrize("norm", [True, False])
def test_qkv_rope_cache_vs_oracle(M, Hq, Hkv, norm):
    from kernels.attention_fused import BlockKVCache, qkv_rope_cache
    print(f"qkv_rope_cache M={M} Hq={Hq} Hkv={Hkv} norm={norm}", flush=True)
    qkv, qn, kn, cos, sin = _qkv_case(M, Hq, Hkv, 4096, seed=M * 3 + Hq)
    if not norm:
        qn = kn = None
    cache = BlockKVCache(2, Hkv, 512, 64, DEV)
    before_k = cache.keys(1)
    pos = torch.randperm(4096, device=DEV)[:M]
    perm = torch.randperm(cache.full_len, device=DEV)      # two disjoint slot sets
    slots, slots2 = perm[:M], perm[M:2 * M]
    with torch.inference_mode():
        q = qkv_rope_cache(qkv, Hq, qn, kn, 1e-6, cos, sin, pos, slots, cache, 1, slots2=slots2)
    torch.cuda.synchronize()
    rq, rk, rv = _oracle_qkv(qkv, Hq, Hkv, qn, kn, cos, sin, pos)
    _close_ulp(q.float().cpu().numpy(), rq)
    kc = cache.keys(1).float().cpu().numpy()
    vc = cache.values(1).float().cpu().numpy()
    for sl in (slots, slots2):
        s = sl.cpu().numpy()
        _close_ulp(kc[:, s].transpose(1, 0, 2), rk)
        assert np.array_equal(vc[:, s].transpose(1, 0, 2), rv)
    touched = set(slots.cpu().tolist()) | set(slots2.cpu().tolist())
    untouched = [i for i in range(cache.full_len) if i not in touched]
    assert torch.equal(cache.keys(1)[:, untouched], before_k[:, untouched])
    assert torch.count_nonzero(cache.values(1)[:, untouched]) == 0
    assert torch.count_nonzero(cache.k_tiles[0]) == 0 and torch.count_nonzero(cache.v_tiles[0]) == 0


def test_qkv_rope_cache_bad_positions_and_slots():
    from kernels.attention_fused import BlockKVCache, qkv_rope_cache
    qkv, qn, kn, cos, sin = _qkv_case(3, 8, 4, 100, seed=5)
    cache = BlockKVCache(1, 4, 64, 32, DEV)
    pos = torch.tensor([5, 100, -1], device=DEV)            # rows 1, 2 out of range
    slots = torch.tensor([3, 4, cache.full_len], device=DEV)  # the last slot is out of range
    with torch.inference_mode():
        q = qkv_rope_cache(qkv, 8, qn, kn, 1e-6, cos, sin, pos, slots, cache, 0)
    assert torch.count_nonzero(q[1:]) == 0
    assert torch.count_nonzero(cache.keys(0)[:, 4]) == 0   # no k write for a bad position
    assert torch.count_nonzero(cache.values(0)[:, 4]) > 0   # v is still written
    assert torch.count_nonzero(cache.keys(0)[:, 3]) > 0
    assert torch.count_nonzero(cache.keys(0)[:, 5:]) == 0 and torch.count_nonzero(cache.values(0)[:, 5:]) == 0


def test_reference_sequence_end_to_end():
    """qkv_rope_cache + block_attention against the reference's torch sequence
    (stock norms, apply_rotary_pos_emb, GQA-expanded index_copy_ writes, SDPA
    with the bool mask) for one verify-shaped forward: 32 scratch rows over a
    600-slot context."""
    from kernels.attention_fused import BlockKVCache, block_attention, qkv_rope_cache
    M, Hq, Hkv, ctx = 32, 32, 8, 600
    n_rep = Hq // Hkv
    qkv, qn, kn, cos, sin = _qkv_case(M, Hq, Hkv, 4096, seed=31)
    cache = BlockKVCache(1, Hkv, 640, M, DEV)
    k_ctx, v_ctx = fill_cache(cache, 0, ctx, seed=40)
    pos = torch.arange(ctx, ctx + M, device=DEV)
    slots = torch.arange(cache.max_cache_len, cache.max_cache_len + M, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(9)
    mask = torch.zeros(M, cache.full_len, dtype=torch.bool, device=DEV)
    mask[:, :ctx] = True
    mask[:, cache.max_cache_len:cache.max_cache_len + M] = torch.rand(M, M, generator=g, device=DEV) < 0.5
    mask[torch.arange(M), cache.max_cache_len + torch.arange(M, device=DEV)] = True
    with torch.inference_mode():
        q = qkv_rope_cache(qkv, Hq, qn, kn, 1e-6, cos, sin, pos, slots, cache, 0)
        out = block_attention(q, cache, 0, mask=mask).view(M, Hq, D)
    # the reference, in torch on the device (SDPA in fp32)
    x = qkv.view(M, Hq + 2 * Hkv, D)
    c, s = cos[pos], sin[pos]

    def norm_rope(t, w):
        t32 = t.float()
        t = w * (t32 * torch.rsqrt(t32.pow(2).mean(-1, keepdim=True) + 1e-6)).to(t.dtype)
        t1, t2 = t[..., :64], t[..., 64:]
        return (t * c[:, None]) + (torch.cat((-t2, t1), dim=-1) * s[:, None])

    qr = norm_rope(x[:, :Hq], qn)
    kr = norm_rope(x[:, Hq:Hq + Hkv], kn)
    vr = x[:, Hq + Hkv:]
    kexp = torch.zeros(1, Hq, cache.full_len, D, device=DEV, dtype=torch.bfloat16)
    vexp = torch.zeros_like(kexp)
    for i in range(n_rep):
        kexp[:, i::n_rep, :ctx] = k_ctx[None]
        vexp[:, i::n_rep, :ctx] = v_ctx[None]
        kexp[:, i::n_rep].index_copy_(2, slots, kr.transpose(0, 1)[None])
        vexp[:, i::n_rep].index_copy_(2, slots, vr.transpose(0, 1)[None])
    ref = F.scaled_dot_product_attention(qr.transpose(0, 1)[None].float(), kexp.float(), vexp.float(),
                                         attn_mask=mask[None, None], scale=D ** -0.5)[0].transpose(0, 1)
    err = float((out.float() - ref).abs().max())
    assert err <= 2 ** -7 * float(ref.abs().max()) + 1e-3, err


@pytest.mark.parametrize("max_cache,n_ctx", [(224, 200), (480, 400), (2016, 900)])
def test_graph_capture_replays(max_cache, n_ctx):
    """Replays of a captured norm + RoPE + cache write + attention equal eager
    calls: one workgroup per KV head (256 slots) and the split form with its
    arrival counters (512 and 2048 slots)."""
    from kernels.attention_fused import BlockKVCache, block_attention, qkv_rope_cache
    M, Hq, Hkv = 4, 16, 8
    qkv, qn, kn, cos, sin = _qkv_case(M, Hq, Hkv, 2048, seed=50)
    cache = BlockKVCache(1, Hkv, max_cache, 32, DEV)
    fill_cache(cache, 0, n_ctx, seed=51)
    pos = torch.arange(n_ctx, n_ctx + 4, device=DEV)
    slots = torch.arange(max_cache, max_cache + 4, device=DEV)
    mask = torch.zeros(M, cache.full_len, dtype=torch.bool, device=DEV)
    mask[:, :n_ctx] = True
    mask[:, max_cache:max_cache + 4] = True
    with torch.inference_mode():
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            block_attention(qkv_rope_cache(qkv, Hq, qn, kn, 1e-6, cos, sin, pos, slots, cache, 0), cache, 0, mask)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = block_attention(qkv_rope_cache(qkv, Hq, qn, kn, 1e-6, cos, sin, pos, slots, cache, 0),
                                  cache, 0, mask)
        for r in range(3):
            qkv.copy_(rnd(M, (Hq + 2 * Hkv) * D, scale=2.0, seed=60 + r))
            g.replay()
            torch.cuda.synchronize()
            ref = block_attention(qkv_rope_cache(qkv, Hq, qn, kn, 1e-6, cos, sin, pos, slots, cache, 0),
                                  cache, 0, mask)
            torch.cuda.synchronize()
            assert torch.equal(out, ref)


@pytest.mark.parametrize("M,Hq,Hkv,L_host,L_dev", [(4, 16, 8, 1500, 700), (16, 16, 8, 1100, 333),
                                                   (4, 16, 8, 3000, 2500), (4, 16, 8, 900, 0),
                                                   (4, 16, 8, 1200, 45), (16, 16, 8, 2000, 100),
                                                   (4, 16, 8, 5000, 4500), (16, 32, 8, 3000, 1000),
                                                   (36, 32, 8, 1200, 500), (36, 32, 8, 1000, 200)])
def test_valid_len_dev_lowers_the_range(M, Hq, Hkv, L_host, L_dev):
    """A device-side valid length below the host's bound gives the attention
    over [0, L_dev) (rows see nothing when it is 0), on both the one-launch
    and the chunked path."""
    from kernels.attention_fused import BlockKVCache, block_attention
    print(f"valid_len_dev M={M} L_host={L_host} L_dev={L_dev}", flush=True)
    cache = BlockKVCache(1, Hkv, L_host, 32, DEV)
    k, v = fill_cache(cache, 0, L_host, seed=L_dev + 3)
    q = rnd(M, Hq, D, seed=8)
    lv = torch.tensor([L_dev], dtype=torch.int64, device=DEV)
    with torch.inference_mode():
        out = block_attention(q, cache, 0, valid_len=L_host, valid_len_dev=lv)
    got = out.view(M, Hq, D).float().cpu().numpy()
    if L_dev == 0:
        assert np.all(got == 0)
        return
    ref = oatt.attention(q.float().cpu().numpy(), k[:, :L_dev].float().cpu().numpy(),
                         v[:, :L_dev].float().cpu().numpy(), None, D ** -0.5)
    assert float(np.abs(got - ref).max()) <= bound(ref)


def test_split_head_counters_stay_zero_across_forms():
    """Calls of every form share the cache's workspace: the split head form's
    arrival counters are back at zero after each call, and each call repeats
    its first result bit for bit whatever ran before it -- the draft's 4
    tokens x 2 query heads per KV head (head or chunked form) and the verify's
    36 x 4 (chunked form)."""
    from kernels.attention_fused import BlockKVCache, block_attention
    Hkv = 8
    cache = BlockKVCache(1, Hkv, 4992, 32, DEV)
    k, v = fill_cache(cache, 0, 5024, seed=70)
    qs = {4: rnd(4, 16, D, seed=71), 36: rnd(36, 32, D, seed=72)}
    first = {}
    with torch.inference_mode():
        for rep in range(3):
            for M, L in ((4, 5000), (36, 1000), (4, 1000), (36, 5000), (4, 2000), (36, 200), (4, 200),
                         (36, 2100), (4, 1500), (4, 5024)):
                print(f"split counters rep={rep} M={M} L={L}", flush=True)
                q = qs[M]
                out = block_attention(q, cache, 0, valid_len=L).clone()
                torch.cuda.synchronize()
                counters = cache._attn_ws[:4 * Hkv].view(torch.int32)
                assert int(counters.abs().sum()) == 0
                if (M, L) not in first:
                    first[M, L] = out
                    ref = oatt.attention(q.float().cpu().numpy(), k[:, :L].float().cpu().numpy(),
                                         v[:, :L].float().cpu().numpy(), None, D ** -0.5)
                    got = out.view(M, q.shape[1], D).float().cpu().numpy()
                    assert float(np.abs(got - ref).max()) <= bound(ref)
                else:
                    assert torch.equal(out, first[M, L])


def test_errors():
    from kernels.attention_fused import BlockKVCache, block_attention, qkv_rope_cache
    cache = BlockKVCache(1, 8, 64, 32, DEV)
    with pytest.raises(TypeError):
        block_attention(rnd(4, 16, D, dtype=torch.float32), cache, 0)
    with pytest.raises(ValueError):
        block_attention(rnd(4, 12, D), cache, 0)             # 12 heads over 8 KV heads
    with pytest.raises(ValueError):
        block_attention(rnd(4, 16, D), cache, 0, valid_len=cache.full_len + 1)
    qkv, qn, kn, cos, sin = _qkv_case(2, 16, 8, 64, seed=1)
    with pytest.raises(ValueError):
        qkv_rope_cache(qkv[:, :-128], 16, qn, kn, 1e-6, cos, sin, torch.zeros(2, dtype=torch.int64, device=DEV),
                       torch.zeros(2, dtype=torch.int64, device=DEV), cache, 0)


@pytest.mark.parametrize("M,Hq,Hkv,ctx", [(4, 16, 8, 1020), (8, 16, 8, 500), (4, 16, 8, 100), (8, 32, 8, 700),
                                          (16, 16, 8, 2000), (1, 16, 8, 3000), (5, 10, 5, 63), (4, 16, 8, 4088),
                                          (2, 16, 8, 0), (7, 8, 8, 384),
                                          # 8-wide grids, whose roles rotate by the KV head
                                          (4, 16, 8, 1396), (8, 16, 8, 1300), (8, 32, 8, 1400)])
@pytest.mark.parametrize("masked", [False, True])
def test_qkv_rope_attention_vs_oracle(M, Hq, Hkv, ctx, masked):
    """The fused launch (q/k norm + RoPE + cache write + attention, the rows at
    the last M slots of the valid range) against the oracle -- the queries and
    new keys normed and rotated, attention over the context and the new rows
    -- within the reference's bf16 bound; the cache's new K within one bf16
    step of the oracle's and its new V exact; every other slot untouched; the
    same call as the two-launch pair within the bound.  The device-side valid
    length sits below the host's bound."""
    from kernels.attention_fused import (BlockKVCache, block_attention, fused_attention_ok, qkv_rope_attention,
                                         qkv_rope_cache)
    print(f"qkv_rope_attention M={M} Hq={Hq} Hkv={Hkv} ctx={ctx} masked={masked}", flush=True)
    valid = ctx + M
    host_bound = min(4096, valid + 40)
    assert fused_attention_ok(M, Hq, Hkv, host_bound)
    qkv, qn, kn, cos, sin = _qkv_case(M, Hq, Hkv, 8192, seed=M * 5 + ctx)
    caches = [BlockKVCache(1, Hkv, (valid + 63) // 32 * 32 + 32, 32, DEV) for _ in range(2)]
    for c in caches:
        k_ctx, v_ctx = fill_cache(c, 0, ctx, seed=ctx + 7) if ctx else (None, None)
    before_k, before_v = caches[0].keys(0).clone(), caches[0].values(0).clone()
    pos = torch.randperm(8192, device=DEV)[:M]
    slots = torch.arange(ctx, valid, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(13)
    full = caches[0].full_len
    mask = torch.zeros(M, full, dtype=torch.bool, device=DEV)
    mask[:, :ctx] = True
    mask[:, ctx:valid] = torch.tril(torch.ones(M, M, dtype=torch.bool, device=DEV))
    if masked:
        mask[:, :valid] &= torch.rand(M, valid, generator=g, device=DEV) < 0.7
        mask[:, ctx] = True
        if M > 2:
            mask[1] = False                     # a row with nothing visible -> zeros
    vdev = torch.tensor([valid], dtype=torch.int64, device=DEV)
    with torch.inference_mode():
        out = qkv_rope_attention(qkv, Hq, qn, kn, 1e-6, cos, sin, pos, caches[0], 0, mask, valid_len=host_bound,
                                 valid_len_dev=vdev).view(M, Hq, D)
        q2 = qkv_rope_cache(qkv, Hq, qn, kn, 1e-6, cos, sin, pos, slots, caches[1], 0)
        pair = block_attention(q2, caches[1], 0, mask, valid_len=host_bound, valid_len_dev=vdev).view(M, Hq, D)
        again = qkv_rope_attention(qkv, Hq, qn, kn, 1e-6, cos, sin, pos, caches[0], 0, mask,
                                   valid_len=host_bound, valid_len_dev=vdev).view(M, Hq, D)
    torch.cuda.synchronize()
    assert torch.equal(out, again)                           # deterministic, and idempotent on the cache
    rq, rk, rv = _oracle_qkv(qkv, Hq, Hkv, qn, kn, cos, sin, pos)
    kc = caches[0].keys(0).float().cpu().numpy()
    vc = caches[0].values(0).float().cpu().numpy()
    # the new K: the norm's statistic is summed in another order than the
    # oracle's (and than qkv_rope_cache's), so a row's scale may round the
    # other way; RoPE's sum of two rounded terms can cancel, so the bound is
    # one bf16 step of the row's largest value, not of each value
    kn_got = kc[:, ctx:valid].transpose(1, 0, 2)
    assert np.all(np.abs(kn_got - rk) <= 2.0 ** -7 * np.abs(rk).max(axis=-1, keepdims=True))
    assert (kn_got != rk).mean() < 0.02
    assert np.array_equal(vc[:, ctx:valid].transpose(1, 0, 2), rv)
    others = [i for i in range(full) if not ctx <= i < valid]
    assert torch.equal(caches[0].keys(0)[:, others], before_k[:, others])
    assert torch.equal(caches[0].values(0)[:, others], before_v[:, others])
    k_all = kc[:, :valid]
    v_all = vc[:, :valid]
    ref = oatt.attention(rq, k_all, v_all, mask[:, :valid].cpu().numpy(), D ** -0.5)
    got = out.float().cpu().numpy()
    err = float(np.abs(got - ref).max())
    assert err <= bound(ref), f"fused: max err {err:.3e} > {bound(ref):.3e}"
    assert float(np.abs(pair.float().cpu().numpy() - got).max()) <= bound(ref)
    if masked and M > 2:
        assert np.all(got[1] == 0)


def test_qkv_rope_attention_graph_replays():
    """Replays of a captured fused launch over a growing device-side valid
    length (the runner's use) equal eager calls at each length."""
    from kernels.attention_fused import BlockKVCache, qkv_rope_attention
    M, Hq, Hkv, base = 4, 16, 8, 900
    qkv, qn, kn, cos, sin = _qkv_case(M, Hq, Hkv, 4096, seed=70)
    cache = BlockKVCache(1, Hkv, 1024, 32, DEV)
    fill_cache(cache, 0, 1000, seed=71)
    ref_cache = BlockKVCache(1, Hkv, 1024, 32, DEV)
    fill_cache(ref_cache, 0, 1000, seed=71)
    pos = torch.zeros(M, dtype=torch.int64, device=DEV)
    vdev = torch.zeros(1, dtype=torch.int64, device=DEV)
    mask = torch.ones(M, cache.full_len, dtype=torch.bool, device=DEV)
    with torch.inference_mode():
        def body():
            return qkv_rope_attention(qkv, Hq, qn, kn, 1e-6, cos, sin, pos, cache, 0, mask, valid_len=1024,
                                      valid_len_dev=vdev)
        pos.copy_(torch.arange(base, base + M, device=DEV))
        vdev.fill_(base + M)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            body()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = body()
        for step in range(4):
            start = base + 8 * step
            pos.copy_(torch.arange(start, start + M, device=DEV))
            vdev.fill_(start + M)
            qkv.copy_(rnd(M, (Hq + 2 * Hkv) * D, scale=2.0, seed=80 + step))
            g.replay()
            torch.cuda.synchronize()
            want = qkv_rope_attention(qkv, Hq, qn, kn, 1e-6, cos, sin, pos, ref_cache, 0, mask, valid_len=1024,
                                      valid_len_dev=vdev)
            assert torch.equal(out, want), step
            assert torch.equal(cache.keys(0), ref_cache.keys(0)) and torch.equal(cache.values(0), ref_cache.values(0))


@pytest.mark.parametrize("M,Hq,Hkv,L_valid", [(4, 16, 8, 1024), (8, 16, 8, 600), (16, 16, 8, 300),
                                              (8, 32, 8, 2048), (1, 16, 8, 64)])
def test_qkv_rope_attention_gathered_tables_equal_positions(M, Hq, Hkv, L_valid):
    """The rows' cos / sin gathered once (position_ids=None, the decoder's
    forwards) give exactly the output and cache writes of the position form,
    from separate tables and from the interleaved pair (one gather)."""
    from kernels.attention_fused import BlockKVCache, gather_rope_rows, qkv_rope_attention, rope_table_pair
    print(f"gathered rope rows: M={M} Hq={Hq} Hkv={Hkv} L={L_valid}", flush=True)
    qkv, qn, kn, cos, sin = _qkv_case(M, Hq, Hkv, 4096, seed=90 + M)
    pos = torch.arange(L_valid - M, L_valid, device=DEV)
    pos[0] = 7                                               # positions need not follow the slots
    mask = torch.ones(M, L_valid + 32, dtype=torch.bool, device=DEV)
    caches = [BlockKVCache(1, Hkv, L_valid, 32, DEV) for _ in range(3)]
    for c in caches:
        fill_cache(c, 0, L_valid - M, seed=91)
    pc, ps = rope_table_pair(cos, sin)
    with torch.inference_mode():
        want = qkv_rope_attention(qkv, Hq, qn, kn, 1e-6, cos, sin, pos, caches[0], 0, mask, valid_len=L_valid)
        got1 = qkv_rope_attention(qkv, Hq, qn, kn, 1e-6, *gather_rope_rows(cos, sin, pos), None, caches[1], 0,
                                  mask, valid_len=L_valid)
        rows = gather_rope_rows(pc, ps, pos)
        got2 = qkv_rope_attention(qkv, Hq, qn, kn, 1e-6, *rows, None, caches[2], 0, mask, valid_len=L_valid)
    torch.cuda.synchronize()
    assert rows[0].stride(0) == 2 * D                        # one gather of the interleaved pair
    for got, c in ((got1, caches[1]), (got2, caches[2])):
        assert torch.equal(got, want)
        assert torch.equal(c.k_tiles[0], caches[0].k_tiles[0]) and torch.equal(c.v_tiles[0], caches[0].v_tiles[0])
