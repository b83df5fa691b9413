"""GPU parity of the x-packed layout (vLLM reshape_and_cache +
paged_attention_v1/v2 as the reference's dense sandbox calls them): the append
is bit-exact against the oracle; attention is within max-abs 2e-2 / mean-abs
2e-3, and v2's partition scratch matches the oracle's per-partition values."""
import numpy as np
import pytest
import torch

from gpu_offloading_amd import ops
from helpers import assert_attn_close, u16
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu


def _dt(name):
    return torch.float16 if name == "fp16" else torch.bfloat16


def _caches(nb, h, dtype, gen, device):
    kc = torch.randn(nb, h, 16, 16, 8, generator=gen, device=device).to(dtype)
    vc = torch.randn(nb, h, 128, 16, generator=gen, device=device).to(dtype)
    return kc, vc


@pytest.mark.parametrize("dt", ["fp16", "bf16"])
def test_xpacked_append_bit_exact(gpu, dt):
    """K/V are strided views of a packed qkv [N, 3, H, D] tensor, as in the
    sandbox; -1 slots are skipped, out-of-range ones counted."""
    g = torch.Generator(device=gpu).manual_seed(60)
    h, nb, n = 8, 40, 300
    kc, vc = _caches(nb, h, _dt(dt), g, gpu)
    qkv = torch.randn(n, 3, h, 128, generator=g, device=gpu).to(_dt(dt))
    k, v = qkv[:, 1], qkv[:, 2]
    slots = torch.randperm(nb * 16, generator=torch.Generator().manual_seed(61))[:n].to(torch.int64)
    slots[5] = -1
    slots[9] = nb * 16 + 3
    k_ref, v_ref = u16(kc).copy(), u16(vc).copy()
    oob = torch.zeros(1, dtype=torch.int32, device=gpu)
    ops.reshape_and_cache(k, v, kc, vc, slots.to(gpu), "auto", oob_count=oob)
    torch.cuda.synchronize()
    orc.reshape_and_cache_xpacked(u16(k.contiguous()), u16(v.contiguous()), k_ref, v_ref,
                                  slots.numpy())
    assert np.array_equal(u16(kc), k_ref) and np.array_equal(u16(vc), v_ref)
    assert int(oob.item()) == 1


def test_xpacked_append_whole_blocks_bit_exact(gpu):
    """Prefill-style slots (16 consecutive tokens filling one block, in
    order) take the LDS-transposed V path; a trailing partial group and a
    group straddling two blocks take the element path.  Both bit-exact."""
    g = torch.Generator(device=gpu).manual_seed(67)
    h, nb = 6, 30
    kc, vc = _caches(nb, h, torch.bfloat16, g, gpu)
    blocks = torch.randperm(nb, generator=torch.Generator().manual_seed(68))[:13]
    ar = torch.arange(16)
    slots = torch.cat([(blocks[:10, None] * 16 + ar).reshape(-1),       # 10 whole blocks
                       blocks[10] * 16 + ar[8:], blocks[11] * 16 + ar[:8],  # straddles two
                       blocks[12] * 16 + ar[:5],                          # partial group,
                       blocks[12] * 16 + torch.tensor([9, 12])])          # out of order
    n = slots.numel()
    k = torch.randn(n, h, 128, generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn(n, h, 128, generator=g, device=gpu).to(torch.bfloat16)
    k_ref, v_ref = u16(kc).copy(), u16(vc).copy()
    ops.reshape_and_cache(k, v, kc, vc, slots.to(torch.int64).to(gpu), "auto")
    torch.cuda.synchronize()
    orc.reshape_and_cache_xpacked(u16(k), u16(v), k_ref, v_ref, slots.numpy())
    assert np.array_equal(u16(kc), k_ref) and np.array_equal(u16(vc), v_ref)


def _attn_case(lens, hq, hkv, dt, seed, gpu, nb_extra=8):
    g = torch.Generator(device=gpu).manual_seed(seed)
    need = sum((n + 15) // 16 for n in lens)
    nb = need + nb_extra
    kc, vc = _caches(nb, hkv, _dt(dt), g, gpu)
    cols = max(1, max((n + 15) // 16 for n in lens))
    bt = np.full((len(lens), cols), -1, np.int32)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed + 1)).numpy()
    at = 0
    for b, n in enumerate(lens):
        k = (n + 15) // 16
        bt[b, :k] = perm[at:at + k]
        at += k
    q = torch.randn(len(lens), hq, 128, generator=g, device=gpu).to(_dt(dt))
    return q, kc, vc, bt


def _run_v2(q, kc, vc, bt, lens, hkv, scale, gpu, max_seq_len=None):
    max_seq_len = max_seq_len or max(max(lens), 1)
    parts = (max_seq_len + 511) // 512
    out = torch.empty_like(q)
    es = torch.empty(q.shape[0], q.shape[1], parts, device=gpu)
    ml = torch.empty_like(es)
    tmp = torch.empty(q.shape[0], q.shape[1], parts, 128, dtype=q.dtype, device=gpu)
    ops.paged_attention_v2(out, es, ml, tmp, q, kc, vc, hkv, scale, torch.from_numpy(bt).to(gpu),
                           torch.tensor(lens, dtype=torch.int32, device=gpu), 16, max_seq_len,
                           None, "auto", torch.tensor(1.0), torch.tensor(1.0), 0, 0, 0, 0, 0)
    torch.cuda.synchronize()
    return out, es, ml, tmp


@pytest.mark.parametrize("dt", ["fp16", "bf16"])
def test_xpacked_v2_matches_oracle_with_partition_scratch(gpu, dt):
    lens = [1, 17, 511, 512, 513, 1500, 3000]
    q, kc, vc, bt = _attn_case(lens, 32, 32, dt, 62, gpu)
    scale = 1 / np.sqrt(128)
    out, es, ml, tmp = _run_v2(q, kc, vc, bt, lens, 32, scale, gpu)
    ref, rml, res, rtmp = orc.paged_attention_xpacked(u16(q), u16(kc), u16(vc), bt,
                                                      np.array(lens), scale, dtype=dt)
    assert_attn_close(out.float().cpu().numpy(), ref)
    for b, n in enumerate(lens):
        P = (n + 511) // 512
        assert np.abs(ml.cpu().numpy()[b, :, :P] - rml[b, :, :P]).max() < 2e-3
        rel = np.abs(es.cpu().numpy()[b, :, :P] / res[b, :, :P] - 1).max()
        assert rel < 2e-3, rel
        assert_attn_close(tmp.float().cpu().numpy()[b, :, :P], rtmp[b, :, :P])


@pytest.mark.parametrize("dt,group", [("fp16", 1), ("bf16", 2), ("bf16", 4), ("fp16", 8)])
def test_xpacked_v1_and_gqa(gpu, dt, group):
    lens = [5, 100, 700, 2049]
    hkv = 4
    q, kc, vc, bt = _attn_case(lens, hkv * group, hkv, dt, 63 + group, gpu)
    scale = 0.07
    out = torch.empty_like(q)
    ops.paged_attention_v1(out, q, kc, vc, hkv, scale, torch.from_numpy(bt).to(gpu),
                           torch.tensor(lens, dtype=torch.int32, device=gpu), 16, max(lens),
                           None, "auto", 1.0, 1.0)
    torch.cuda.synchronize()
    ref, *_ = orc.paged_attention_xpacked(u16(q), u16(kc), u16(vc), bt, np.array(lens), scale,
                                          dtype=dt)
    assert_attn_close(out.float().cpu().numpy(), ref)
    out2, *_ = _run_v2(q, kc, vc, bt, lens, hkv, scale, gpu)
    assert_attn_close(out2.float().cpu().numpy(), ref)


def test_xpacked_random_shapes(gpu):
    """Seeded random batches, v1 and v2 against the oracle: fp16 / bf16,
    group sizes 1-8, 1-16 KV heads, 1-20 sequences of 0-3000 tokens (empty
    ones give zeros), and v2 launched with a max_seq_len up to 1500 tokens
    past the longest sequence (partitions no sequence reaches)."""
    rng = np.random.default_rng(53)
    for case in range(16):
        dt = ["fp16", "bf16"][case % 2]
        group = int(rng.choice([1, 2, 4, 8]))
        hkv = int(rng.choice([1, 2, 4, 8, 16]))
        b = int(rng.integers(1, 21))
        lens = np.where(rng.random(b) < 0.1, 0, rng.integers(1, 3001, b))
        while int(lens.sum()) * hkv > 400_000:
            lens = (lens + 1) // 2
        lens = [int(x) for x in lens]
        scale = float(rng.uniform(0.03, 0.12))
        extra = int(rng.integers(0, 1501))
        print(f"xpacked random case {case}: {dt} G={group} Hkv={hkv} lens={lens} extra={extra}",
              flush=True)
        q, kc, vc, bt = _attn_case(lens, hkv * group, hkv, dt, 400 + case, gpu)
        ref, *_ = orc.paged_attention_xpacked(u16(q), u16(kc), u16(vc), bt, np.array(lens), scale,
                                              dtype=dt)
        live = [i for i, n in enumerate(lens) if n]
        empty = [i for i, n in enumerate(lens) if not n]
        out1 = torch.empty_like(q)
        ops.paged_attention_v1(out1, q, kc, vc, hkv, scale, torch.from_numpy(bt).to(gpu),
                               torch.tensor(lens, dtype=torch.int32, device=gpu), 16,
                               max(max(lens), 1), None, "auto", 1.0, 1.0)
        out2, *_ = _run_v2(q, kc, vc, bt, lens, hkv, scale, gpu,
                           max_seq_len=max(max(lens), 1) + extra)
        for out in (out1, out2):
            if live:
                assert_attn_close(out[live].float().cpu().numpy(), ref[live])
            if empty:
                assert (out[empty] == 0).all()


def test_xpacked_empty_sequence_and_nan_past_the_end(gpu):
    lens = [0, 37, 600]
    q, kc, vc, bt = _attn_case(lens, 8, 8, "fp16", 64, gpu)
    last = int(bt[1, 2])
    kc[last, :, :, 37 % 16:] = float("nan")
    vc[last, :, :, 37 % 16:] = float("nan")
    out, *_ = _run_v2(q, kc, vc, bt, lens, 8, 0.09, gpu)
    assert torch.isfinite(out).all() and (out[0] == 0).all()
    ref, *_ = orc.paged_attention_xpacked(u16(q), u16(kc), u16(vc), bt, np.array(lens), 0.09)
    assert_attn_close(out[1:].float().cpu().numpy(), ref[1:])


def test_xpacked_append_then_attention_equals_flat_layout_decode(gpu):
    """Same tokens appended to both layouts: paged_attention_v2 on the
    x-packed cache agrees with the flat-layout decode kernel."""
    from gpu_offloading_amd.decode import BatchDecodeWithPagedKVCacheWrapper

    g = torch.Generator(device=gpu).manual_seed(65)
    lens, h = [300, 41, 1030], 8
    nb = 120
    n = sum(lens)
    key = torch.randn(n, h, 128, generator=g, device=gpu).to(torch.bfloat16)
    val = torch.randn(n, h, 128, generator=g, device=gpu).to(torch.bfloat16)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(66)).numpy()
    bt = np.full((3, 65), -1, np.int32)
    at = 0
    slots = []
    for b, ln in enumerate(lens):
        k = (ln + 15) // 16
        bt[b, :k] = perm[at:at + k]
        at += k
        pos = np.arange(ln)
        slots.append(bt[b, pos // 16].astype(np.int64) * 16 + pos % 16)
    slots = torch.from_numpy(np.concatenate(slots)).to(gpu)
    kx = torch.zeros(nb, h, 16, 16, 8, dtype=torch.bfloat16, device=gpu)
    vx = torch.zeros(nb, h, 128, 16, dtype=torch.bfloat16, device=gpu)
    kf = torch.zeros(nb, 16, h, 128, dtype=torch.bfloat16, device=gpu)
    vf = torch.zeros_like(kf)
    ops.reshape_and_cache(key, val, kx, vx, slots)
    ops.reshape_and_cache_flash(key, val, kf, vf, slots)
    q = torch.randn(3, h, 128, generator=g, device=gpu).to(torch.bfloat16)
    out, *_ = _run_v2(q, kx, vx, bt, lens, h, 1 / np.sqrt(128), gpu)
    indptr, lpl = orc.plan_decode(lens)
    idx = orc.page_indices(bt, range(3), indptr)
    w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(1 << 26, dtype=torch.uint8, device=gpu))
    w.plan(torch.from_numpy(indptr), torch.from_numpy(idx).to(gpu), torch.from_numpy(lpl),
           num_qo_heads=h, num_kv_heads=h, head_dim=128, page_size=16)
    dout = w.run(q, (kf, vf))
    torch.cuda.synchronize()
    assert_attn_close(out.float().cpu().numpy(), dout.float().cpu().numpy())


def test_xpacked_rejects_bad_inputs(gpu):
    kc = torch.zeros(4, 2, 16, 16, 8, dtype=torch.float16, device=gpu)
    vc = torch.zeros(4, 2, 128, 16, dtype=torch.float16, device=gpu)
    q = torch.zeros(1, 2, 128, dtype=torch.float16, device=gpu)
    bt = torch.zeros(1, 4, dtype=torch.int32, device=gpu)
    sl = torch.tensor([20], dtype=torch.int32, device=gpu)
    out = torch.empty_like(q)
    es = torch.empty(1, 2, 1, device=gpu)
    with pytest.raises(RuntimeError, match="partitions"):
        ops.paged_attention_v2(out, es, es.clone(), torch.empty(1, 2, 1, 128, dtype=q.dtype,
                                                                 device=gpu),
                               q, kc, vc, 2, 0.1, bt, sl, 16, 1024)
    with pytest.raises(RuntimeError, match="alibi"):
        ops.paged_attention_v1(out, q, kc, vc, 2, 0.1, bt, sl, 16, 20,
                               alibi_slopes=torch.zeros(2, device=gpu))
    with pytest.raises(RuntimeError, match="block-sparse"):
        ops.paged_attention_v1(out, q, kc, vc, 2, 0.1, bt, sl, 16, 20, None, "auto", 1.0, 1.0,
                               0, 4, 0, 64, 0)


def _torch_ref(q, kc, vc, bt, lens, scale):
    """fp32 attention per sequence over the x-packed caches, unpacked on the
    GPU through the layout's closed form (k[tok, h, d] = kc[blk, h, d // 8,
    tok, d % 8]; v[tok, h, d] = vc[blk, h, d, tok])."""
    outs = []
    for b, n in enumerate(lens):
        blocks = torch.from_numpy(bt[b, :(n + 15) // 16].astype(np.int64)).to(q.device)
        k = kc[blocks].permute(0, 3, 1, 2, 4).reshape(-1, kc.shape[1], 128)[:n].float()
        v = vc[blocks].permute(0, 3, 1, 2).reshape(-1, vc.shape[1], 128)[:n].float()
        s = torch.matmul(k.permute(1, 0, 2).contiguous(), q[b].float()[:, :, None])[..., 0] * scale
        p = torch.softmax(s, dim=-1)                                   # [H, n]
        outs.append(torch.matmul(p[:, None, :], v.permute(1, 0, 2).contiguous())[:, 0])
    return torch.stack(outs)


@pytest.mark.parametrize("case", ["1x150000", "64xU512_4096"])
def test_xpacked_at_the_bench_shapes(gpu, case):
    """The benchmark's x-packed shapes (MHA 32 x 128, fp16): one 150,000-token
    sequence (the reference's GH200 point) and 64 sequences of U[512, 4096]
    tokens; v2 (and v1 for the long sequence) against an fp32 reference."""
    rng = np.random.default_rng(64)
    lens = [150_000] if case == "1x150000" else rng.integers(512, 4097, 64).tolist()
    q, kc, vc, bt = _attn_case(lens, 32, 32, "fp16", 65, gpu)
    scale = 1 / np.sqrt(128)
    ref = _torch_ref(q, kc, vc, bt, lens, scale).cpu().numpy()
    out, *_ = _run_v2(q, kc, vc, bt, lens, 32, scale, gpu)
    assert_attn_close(out.float().cpu().numpy(), ref)
    if case == "1x150000":
        out1 = torch.empty_like(q)
        ops.paged_attention_v1(out1, q, kc, vc, 32, scale, torch.from_numpy(bt).to(gpu),
                               torch.tensor(lens, dtype=torch.int32, device=gpu), 16,
                               max(lens), None, "auto", torch.tensor(1.0), torch.tensor(1.0))
        assert_attn_close(out1.float().cpu().numpy(), ref)
