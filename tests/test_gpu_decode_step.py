"""GPU parity: the fused decode step (RoPE on q and k + KV-cache append of k and v).

Reference sequence: WgpuForwardEngine::forward_token / forward_chunk
(crates/sapient-models/src/forward/wgpu_engine.rs:397-432, :527-573) — rope on q
and k (resident.rs:467), then kv_append of k and v (resident.rs:645-711).

Bar: bit-exact against the unfused sequence of this library's own kernels
(sph_rope in place, then sph_kv_append of k and v), whose parity with the oracle
the RoPE and layout tests establish; and q / the caches bit-exact against the
oracle.
"""
import numpy as np
import pytest
import torch

from helpers import to_np, widen
from refvec import WgpuLcg

import sapient_amd.ops as ops

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
IDS = lambda d: str(d).split(".")[-1]


def _gen(shape, seed, dev, dtype):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(shape, generator=g, device=dev).to(dtype)


def _unfused(q, k, v, positions, base, kcache, vcache, interleaved):
    """sph_rope on copies of q and k ([1, H, S, D] views), then one kv_append per token at positions[s]."""
    q2, k2 = q.clone(), k.clone()
    ops.rope_(q2.unsqueeze(0), k2.unsqueeze(0), positions, base, interleaved=interleaved)
    for s, p in enumerate(positions.cpu().tolist()):
        ops.kv_append(k2[:, s:s + 1].contiguous(), kcache, p)
        ops.kv_append(v[:, s:s + 1].contiguous(), vcache, p)
    return q2


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("cdtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "interleaved"])
@pytest.mark.parametrize("Hq,Hkv,S,D,max_seq,pos0", [(14, 2, 1, 64, 64, 37), (32, 8, 512, 128, 1024, 100),
                                                     (32, 32, 3, 80, 16, 13), (4, 2, 5, 8, 12, 0)])
def test_fused_equals_unfused(dev, dtype, cdtype, interleaved, Hq, Hkv, S, D, max_seq, pos0):
    print(f"case rope_kv {dtype} cache {cdtype} {'il' if interleaved else 'neox'} {Hq}+{Hkv}x{S}x{D} pos {pos0}",
          flush=True)
    q = _gen((Hq, S, D), 1, dev, dtype)
    k = _gen((Hkv, S, D), 2, dev, dtype)
    v = _gen((Hkv, S, D), 3, dev, dtype)
    positions = torch.arange(pos0, pos0 + S, dtype=torch.int32, device=dev)
    kc = _gen((Hkv, max_seq, D), 4, dev, cdtype)
    vc = _gen((Hkv, max_seq, D), 5, dev, cdtype)
    kc2, vc2 = kc.clone(), vc.clone()
    k_before = k.clone()
    q_ref = _unfused(q, k, v, positions, 5e5, kc2, vc2, interleaved)
    ops.rope_kv_append(q, k, v, positions, 5e5, kc, vc, interleaved=interleaved)
    assert np.array_equal(to_np(q), to_np(q_ref)), "q"
    assert np.array_equal(to_np(kc), to_np(kc2)), "k cache"
    assert np.array_equal(to_np(vc), to_np(vc2)), "v cache"
    assert torch.equal(k, k_before), "k is read-only"


def test_fused_matches_oracle_and_scatters_by_position(dev, orc):
    """Non-consecutive positions (a shuffled chunk): each token's rows land at its own cache
    row; q and the k cache equal the oracle's apply_rope bit for bit; v is copied."""
    Hq, Hkv, S, D, max_seq = 8, 2, 6, 64, 32
    nxt = WgpuLcg()
    q = nxt.take(Hq * S * D).reshape(Hq, S, D)
    k = nxt.take(Hkv * S * D).reshape(Hkv, S, D)
    v = nxt.take(Hkv * S * D).reshape(Hkv, S, D)
    pos = np.array([9, 3, 30, 0, 17, 4], np.int32)
    tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, k, v))
    kc = torch.zeros(Hkv, max_seq, D, device=dev)
    vc = torch.zeros(Hkv, max_seq, D, device=dev)
    ops.rope_kv_append(tq, tk, tv, torch.from_numpy(pos).to(dev), 1e4, kc, vc)
    want_q = orc.apply_rope(q[None], pos, 1e4)[0]
    want_k = orc.apply_rope(k[None], pos, 1e4)[0]
    bits = lambda a: np.ascontiguousarray(a, np.float32).view(np.uint32)
    assert np.array_equal(bits(to_np(tq)), bits(want_q))
    got_k, got_v = to_np(kc), to_np(vc)
    for s, p in enumerate(pos):
        assert np.array_equal(bits(got_k[:, p]), bits(want_k[:, s]))
        assert np.array_equal(got_v[:, p], v[:, s])
    untouched = np.setdiff1d(np.arange(max_seq), pos)
    assert (got_k[:, untouched] == 0).all() and (got_v[:, untouched] == 0).all()


def test_bad_position_writes_nothing_and_raises_flag(dev):
    Hq, Hkv, S, D, max_seq = 4, 2, 3, 64, 8
    q = _gen((Hq, S, D), 7, dev, torch.float32)
    k = _gen((Hkv, S, D), 8, dev, torch.float32)
    v = _gen((Hkv, S, D), 9, dev, torch.float32)
    kc = torch.zeros(Hkv, max_seq, D, device=dev)
    vc = torch.zeros(Hkv, max_seq, D, device=dev)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    positions = torch.tensor([2, 8, -1], dtype=torch.int32, device=dev)
    q_ref = q.clone()
    ops.rope_(q_ref.unsqueeze(0), None, positions, 1e4)
    ops.rope_kv_append(q, k, v, positions, 1e4, kc, vc, bad_pos_flag=flag)
    assert flag.item() == 1
    assert torch.equal(q, q_ref)  # q rotates at every position
    nz = (kc.abs().sum(dim=(0, 2)) > 0).cpu().tolist()
    assert nz == [False, False, True, False, False, False, False, False]
    assert (vc.abs().sum(dim=(0, 2)) > 0).cpu().tolist() == nz


def test_rejects_bad_arguments(dev):
    from sapient_amd._lib import EINVAL, lib
    L = lib()
    t = torch.zeros(2, 1, 64, device=dev)
    p = torch.zeros(1, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    d = t.data_ptr()
    args = lambda **kw: dict(dict(q=d, hq=2, k=d, v=d, hkv=2, dt=0, lay=0, pos=p.data_ptr(), seq=1, hd=64, base=1e4,
                                  ps=1.0, kc=d, vc=d, cdt=0, ms=1, bq=None, bk=None, bv=None, bdt=0, flag=None,
                                  s=s), **kw)
    call = lambda a: L.sph_rope_kv_append(*a.values())
    assert call(args(hd=63)) == EINVAL                  # odd head_dim
    assert call(args(lay=2)) == EINVAL                  # layout
    assert call(args(cdt=8)) == EINVAL                  # cache dtype
    assert call(args(kc=None)) == EINVAL                # missing cache
    assert call(args(ps=0.0)) == EINVAL                 # pos_scale
    assert call(args(hd=6)) == EINVAL                   # 3 pairs: no vector width divides them
    assert call(args(bq=d, bdt=8)) == EINVAL            # bias dtype


@pytest.mark.parametrize("dtype,cdtype,bdtype", [(torch.float32, torch.float16, torch.float16),
                                                 (torch.float32, torch.float32, torch.float32),
                                                 (torch.float16, torch.float16, torch.float32),
                                                 (torch.bfloat16, torch.float32, torch.bfloat16),
                                                 (torch.float16, torch.bfloat16, torch.bfloat16)], ids=str)
@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "interleaved"])
@pytest.mark.parametrize("Hq,Hkv,S,D", [(14, 2, 1, 64), (32, 8, 37, 128), (4, 2, 5, 8)])
def test_fused_biases_equal_add_bias_then_rope_then_append(dev, dtype, cdtype, bdtype, interleaved, Hq, Hkv, S, D):
    """The projections' bias step (wgpu_engine.rs:397-407, :527-538, sph_add_bias on token-major q/k/v), the
    token-major → heads-major transpose, RoPE and the appends, against the fused call on the
    transposed, bias-free tensors: bit for bit."""
    print(f"case rope_kv bias {dtype} cache {cdtype} bias {bdtype} {'il' if interleaved else 'neox'} "
          f"{Hq}+{Hkv}x{S}x{D}", flush=True)
    max_seq, pos0 = 64, 11
    q_tok = _gen((S, Hq, D), 11, dev, dtype)
    k_tok = _gen((S, Hkv, D), 12, dev, dtype)
    v_tok = _gen((S, Hkv, D), 13, dev, dtype)
    bq = _gen((Hq * D,), 14, dev, bdtype)
    bk = _gen((Hkv * D,), 15, dev, bdtype)
    bv = _gen((Hkv * D,), 16, dev, bdtype)
    positions = torch.arange(pos0, pos0 + S, dtype=torch.int32, device=dev)
    kc = torch.zeros(Hkv, max_seq, D, device=dev, dtype=cdtype)
    vc = torch.zeros(Hkv, max_seq, D, device=dev, dtype=cdtype)
    kc2, vc2 = kc.clone(), vc.clone()
    # unfused: bias in token-major layout, then transpose, RoPE, appends
    qb = ops.add_bias(q_tok.reshape(S, Hq * D), bq).view(S, Hq, D)
    kb = ops.add_bias(k_tok.reshape(S, Hkv * D), bk).view(S, Hkv, D)
    vb = ops.add_bias(v_tok.reshape(S, Hkv * D), bv).view(S, Hkv, D)
    q_ref = _unfused(ops.transpose_heads(qb), ops.transpose_heads(kb), ops.transpose_heads(vb), positions, 1e6,
                     kc2, vc2, interleaved)
    # fused
    q = ops.transpose_heads(q_tok)
    ops.rope_kv_append(q, ops.transpose_heads(k_tok), ops.transpose_heads(v_tok), positions, 1e6, kc, vc,
                       interleaved=interleaved, bq=bq, bk=bk, bv=bv)
    assert np.array_equal(to_np(q), to_np(q_ref)), "q"
    assert np.array_equal(to_np(kc), to_np(kc2)), "k cache"
    assert np.array_equal(to_np(vc), to_np(vc2)), "v cache"


@pytest.mark.parametrize("dtype,cdtype,bdtype", [(torch.float32, torch.float16, None),
                                                 (torch.float32, torch.float32, torch.float32),
                                                 (torch.float32, torch.bfloat16, torch.float16),
                                                 (torch.float16, torch.float16, torch.float32),
                                                 (torch.bfloat16, torch.float32, torch.bfloat16)], ids=str)
@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "interleaved"])
@pytest.mark.parametrize("Hq,Hkv,S,D,pos0", [(14, 2, 512, 64, 0), (32, 8, 37, 128, 100), (4, 2, 5, 8, 3),
                                             (14, 2, 1, 64, 40)])
def test_token_major_variant_equals_transpose_then_fused(dev, dtype, cdtype, bdtype, interleaved, Hq, Hkv, S, D,
                                                         pos0):
    """sph_rope_kv_append_tokens on the projections' token-major q/k/v (the chunk step of
    wgpu_engine.rs:525-573 with its transposes folded in) against sph_transpose_heads of q, k, v and then
    sph_rope_kv_append: q_out, both caches and the flag bit for bit; the inputs are left unchanged."""
    print(f"case rope_kv tokens {dtype} cache {cdtype} bias {bdtype} {'il' if interleaved else 'neox'} "
          f"{Hq}+{Hkv}x{S}x{D} pos {pos0}", flush=True)
    max_seq = pos0 + S + 3
    q_tok = _gen((S, Hq, D), 21, dev, dtype)
    k_tok = _gen((S, Hkv, D), 22, dev, dtype)
    v_tok = _gen((S, Hkv, D), 23, dev, dtype)
    before = [t.clone() for t in (q_tok, k_tok, v_tok)]
    b = {} if bdtype is None else dict(bq=_gen((Hq * D,), 24, dev, bdtype), bk=_gen((Hkv * D,), 25, dev, bdtype),
                                       bv=_gen((Hkv * D,), 26, dev, bdtype))
    positions = torch.arange(pos0, pos0 + S, dtype=torch.int32, device=dev)
    kc = _gen((Hkv, max_seq, D), 27, dev, cdtype)
    vc = _gen((Hkv, max_seq, D), 28, dev, cdtype)
    kc2, vc2 = kc.clone(), vc.clone()
    f1 = torch.zeros(1, dtype=torch.int32, device=dev)
    f2 = torch.zeros(1, dtype=torch.int32, device=dev)
    q_ref = ops.transpose_heads(q_tok)
    ops.rope_kv_append(q_ref, ops.transpose_heads(k_tok), ops.transpose_heads(v_tok), positions, 1e6, kc2, vc2,
                       interleaved=interleaved, bad_pos_flag=f2, **b)
    q_out = ops.rope_kv_append_tokens(q_tok, k_tok, v_tok, positions, 1e6, kc, vc, interleaved=interleaved,
                                      bad_pos_flag=f1, **b)
    assert q_out.shape == (Hq, S, D)
    assert np.array_equal(to_np(q_out), to_np(q_ref)), "q"
    assert np.array_equal(to_np(kc), to_np(kc2)), "k cache"
    assert np.array_equal(to_np(vc), to_np(vc2)), "v cache"
    assert f1.item() == f2.item() == 0
    for t, t0, n in zip((q_tok, k_tok, v_tok), before, "qkv"):
        assert torch.equal(t, t0), f"{n} is read-only"


def test_token_major_variant_rejects_overlap_and_flags_bad_positions(dev):
    from sapient_amd._lib import EINVAL, lib
    S, Hq, Hkv, D, max_seq = 3, 4, 2, 64, 8
    q = _gen((S, Hq, D), 31, dev, torch.float32)
    k = _gen((S, Hkv, D), 32, dev, torch.float32)
    v = _gen((S, Hkv, D), 33, dev, torch.float32)
    kc = torch.zeros(Hkv, max_seq, D, device=dev)
    vc = torch.zeros(Hkv, max_seq, D, device=dev)
    pos = torch.tensor([2, 8, -1], dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    call = lambda qo: lib().sph_rope_kv_append_tokens(q.data_ptr(), qo, Hq, k.data_ptr(), v.data_ptr(), Hkv, 0, 0,
                                                      pos.data_ptr(), S, D, 1e4, 1.0, kc.data_ptr(), vc.data_ptr(),
                                                      0, max_seq, None, None, None, 0, None, s)
    assert call(q.data_ptr()) == EINVAL                 # q_out == q
    assert call(q.data_ptr() + 4 * D) == EINVAL         # partial overlap
    assert call(None) == EINVAL                         # no q_out
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    q_out = ops.rope_kv_append_tokens(q, k, v, pos, 1e4, kc, vc, bad_pos_flag=flag)
    torch.cuda.synchronize()
    assert flag.item() == 1
    q_ref = ops.transpose_heads(q)
    ops.rope_(q_ref.unsqueeze(0), None, pos, 1e4)
    assert torch.equal(q_out, q_ref)  # q rotates at every position
    nz = (kc.abs().sum(dim=(0, 2)) > 0).cpu().tolist()
    assert nz == [False, False, True, False, False, False, False, False]
    assert (vc.abs().sum(dim=(0, 2)) > 0).cpu().tolist() == nz
