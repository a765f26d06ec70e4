"""GPU tests of the device-resident decode engine (include/sapient_hip_engine.h).

Reference sequence: WgpuForwardEngine::forward_token / forward_chunk
(crates/sapient-models/src/forward/wgpu_engine.rs:362-629). Projections and
attention are outside the library, so the tests plug in exactly reproducible
stand-ins, enqueued with torch on the engine's stream:
  projection  out[r, j] = 0.5 · in[r, j mod n_in]   (exact in f32)
  attention   out = q (the rotated queries, heads-major)
and check, in order:
  1. graph replay = eager launches, bit for bit, at every decode step (the
     graph is replayed for several tokens, eager chunks, other work and
     synchronizations in between, also while the RoPE angle table grows);
  2. every op of every layer on the engine's own inputs (the stand-ins record
     what each op received; the residual stream is rebuilt from the records
     with the same f32 adds): the norms to 1e-5 relative, bias + RoPE (NEOX
     and interleaved; the angles come from the host: staged per one-token
     step, rows of a per-position table for a chunk, checked across every
     fill of that table up to max_seq), the KV-cache rows and SwiGLU bit for
     bit;
  3. the end-to-end hidden states and caches against the oracle's run of the
     whole reference sequence on its own values, where the norms' last-bit
     differences compound over the layers: 1e-4 of the largest |value|
     (hidden), one f16 ulp plus that bound (caches);
  4. the engine's refusals (full cache, id ≥ vocab, oversized chunk).
"""
import numpy as np
import pytest
import torch

from helpers import to_np, widen

import sapient_amd._lib as L
from sapient_amd.engine import Engine

pytestmark = pytest.mark.gpu

H, NQ, NKV, HD, INTER, LAYERS, MAX_SEQ, MAX_CHUNK, VOCAB = 256, 8, 2, 32, 512, 3, 64, 16, 100
EPS, THETA = 1e-6, 1e4
PROMPT = [5, 17, 99, 0, 42, 42, 7]
DECODE = [3, 64, 11, 98, 1]
# A prompt, chunks of MAX_CHUNK tokens and single tokens, ending at MAX_SEQ.
STEPS = ([PROMPT, [(7 * i + 3) % VOCAB for i in range(MAX_CHUNK)]] + [[t] for t in DECODE]
         + [[(11 * i + 5) % VOCAB for i in range(MAX_CHUNK)], [8], [13], [21],
            [(13 * i + 1) % VOCAB for i in range(MAX_CHUNK)], [34]])
assert sum(len(s) for s in STEPS) == MAX_SEQ


def _gen(shape, seed, dev, mean=0.0, std=1.0, dtype=torch.float32):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev) * std + mean).to(dtype)


def _n_out(which):
    return {L.PROJ_Q: NQ * HD, L.PROJ_K: NKV * HD, L.PROJ_V: NKV * HD, L.PROJ_O: H, L.PROJ_GATE: INTER,
            L.PROJ_UP: INTER, L.PROJ_DOWN: H}[which]


def _n_in(which):
    return {L.PROJ_O: NQ * HD, L.PROJ_DOWN: INTER}.get(which, H)


def _view(ptr, n):
    from sapient_amd.engine import _DevArray
    return torch.as_tensor(_DevArray(ptr, (n,), "<f4"), device="cuda")


def project(layer, which, in_ptr, out_ptr, rows, stream):
    n_in, n_out = _n_in(which), _n_out(which)
    src = _view(in_ptr, rows * n_in).view(rows, n_in)
    dst = _view(out_ptr, rows * n_out).view(rows, n_out)
    with torch.cuda.stream(torch.cuda.ExternalStream(stream)):
        for j0 in range(0, n_out, n_in):
            w = min(n_in, n_out - j0)
            dst[:, j0:j0 + w].copy_(src[:, :w])
        dst.mul_(0.5)
    return 0


def attend(layer, q_ptr, kc, vc, kv_dtype, pos_ptr, n_tok, max_seq, out_ptr, stream):
    n = NQ * n_tok * HD
    with torch.cuda.stream(torch.cuda.ExternalStream(stream)):
        _view(out_ptr, n).copy_(_view(q_ptr, n))
    return 0


@pytest.fixture(scope="module")
def model(dev):
    table = _gen((VOCAB, H), 1, dev)
    layers = [dict(input_ln=_gen((H,), 10 + l, dev, 1.0, 0.1), post_ln=_gen((H,), 20 + l, dev, 1.0, 0.1),
                   bq=_gen((NQ * HD,), 30 + l, dev, 0.0, 0.1, torch.float16),
                   bk=_gen((NKV * HD,), 40 + l, dev, 0.0, 0.1, torch.float16),
                   bv=_gen((NKV * HD,), 50 + l, dev, 0.0, 0.1, torch.float16), bo=None) for l in range(LAYERS)]
    final = _gen((H,), 60, dev, 1.0, 0.1)
    return table, layers, final


def _engine(model, kv_dtype=L.F16):
    table, layers, final = model
    cfg = L.EngineConfig(H, NQ, NKV, HD, INTER, LAYERS, MAX_SEQ, MAX_CHUNK, EPS, THETA, L.ROPE_NEOX, kv_dtype, L.F16)
    return Engine(cfg, table, L.F32, VOCAB, layers, final, project, attend)


def _run(eng, graph, steps=STEPS):
    eng.use_graph(graph)
    outs = []
    for ids in steps:
        outs.append((eng.forward_chunk(ids) if len(ids) > 1 else eng.forward_token(ids[0])).clone())
        torch.cuda.synchronize()
    return [to_np(o) for o in outs]


def test_graph_replay_equals_eager(dev, model):
    eager = _engine(model)
    e_out = _run(eager, False)
    graph = _engine(model)
    g_out = _run(graph, True)
    print("case engine graph vs eager", flush=True)
    for i, (a, b) in enumerate(zip(e_out, g_out)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {i}"
    for l in range(LAYERS):
        for w in "kv":
            assert torch.equal(eager.cache(l, w), graph.cache(l, w)), f"layer {l} {w} cache"
    assert eager.position == graph.position == MAX_SEQ
    eager.close()
    graph.close()


def _oracle_step(orc, model_np, ids, pos0, caches):
    """One forward call of the reference sequence (wgpu_engine.rs:362-629) with the stand-ins."""
    table, layers, final = model_np
    T = len(ids)
    pos = np.arange(pos0, pos0 + T)
    proj = lambda x, n_out: 0.5 * np.tile(x, (1, -(-n_out // x.shape[1])))[:, :n_out]
    x = orc.embed_tokens(table.reshape(-1).view(np.uint8), L.F32, VOCAB, H, np.array(ids, np.uint32))
    x = x.reshape(T, H)
    down = None
    for l, Lw in enumerate(layers):
        if l > 0:
            x = orc.add(x, down)
        h = orc.rms_norm(x, Lw["input_ln"], EPS)
        q = orc.add_bias_last_dim(proj(h, NQ * HD).astype(np.float32), Lw["bq"])
        k = orc.add_bias_last_dim(proj(h, NKV * HD).astype(np.float32), Lw["bk"])
        v = orc.add_bias_last_dim(proj(h, NKV * HD).astype(np.float32), Lw["bv"])
        qh = q.reshape(T, NQ, HD).transpose(1, 0, 2)[None]
        kh = k.reshape(T, NKV, HD).transpose(1, 0, 2)[None]
        vh = v.reshape(T, NKV, HD).transpose(1, 0, 2)
        qr = orc.apply_rope(np.ascontiguousarray(qh), pos, THETA)[0]
        kr = orc.apply_rope(np.ascontiguousarray(kh), pos, THETA)[0]
        orc.kv_append(kr, caches[l][0], L.F16, NKV, T, HD, MAX_SEQ, pos0)
        orc.kv_append(np.ascontiguousarray(vh), caches[l][1], L.F16, NKV, T, HD, MAX_SEQ, pos0)
        attn = qr.transpose(1, 0, 2).reshape(T, NQ * HD)
        o = proj(attn, H).astype(np.float32)
        x = orc.add(x, o)
        h2 = orc.rms_norm(x, Lw["post_ln"], EPS)
        act = orc.swiglu(proj(h2, INTER).astype(np.float32), proj(h2, INTER).astype(np.float32))
        down = proj(act, H).astype(np.float32)
    last = orc.add(x[-1:], down[-1:])
    return orc.rms_norm(last, final, EPS)[0]


def test_engine_matches_oracle_sequence(dev, orc, model):
    table, layers, final = model
    model_np = (to_np(table), [{k: (None if v is None else widen(v, orc)) for k, v in Lw.items()} for Lw in layers],
                to_np(final))
    eng = _engine(model)
    got = _run(eng, True)
    caches = [(np.zeros((NKV, MAX_SEQ, HD), np.uint16), np.zeros((NKV, MAX_SEQ, HD), np.uint16))
              for _ in range(LAYERS)]
    want, pos0 = [], 0
    for ids in STEPS:
        want.append(_oracle_step(orc, model_np, ids, pos0, caches))
        pos0 += len(ids)
    print("case engine vs oracle", flush=True)
    for i, (g, w) in enumerate(zip(got, want)):
        assert np.abs(g - w).max() <= 1e-4 * np.abs(w).max(), f"step {i}: {np.abs(g - w).max()}"
    used = MAX_SEQ
    for l in range(LAYERS):
        for j, which in enumerate("kv"):
            g = widen(eng.cache(l, which), orc).reshape(NKV, MAX_SEQ, HD)
            w = orc.f16_bits_to_f32(caches[l][j])
            scale = np.abs(w[:, :used]).max()
            assert np.all(np.abs(g[:, :used] - w[:, :used]) <= 2.0 ** -10 * np.abs(w[:, :used]) + 1e-4 * scale), \
                f"layer {l} {which} cache"
    eng.close()


def test_engine_refusals(dev, model):
    from sapient_amd._lib import SapientHipError
    eng = _engine(model)
    with pytest.raises(SapientHipError, match="index out of range"):
        eng.forward_token(VOCAB)
    with pytest.raises(SapientHipError, match="invalid"):
        eng.forward_chunk(list(range(MAX_CHUNK + 1)))
    for _ in range(MAX_SEQ // MAX_CHUNK):
        eng.forward_chunk([1] * MAX_CHUNK)
    assert eng.position == MAX_SEQ
    with pytest.raises(SapientHipError, match="index out of range"):
        eng.forward_token(1)
    eng.reset()
    assert eng.position == 0
    eng.forward_token(2)
    torch.cuda.synchronize()
    eng.close()


class _Recorder:
    """Projection and attention stand-ins (the module's) that also keep each call's input as the engine
    handed it over, so every op of the sequence can be checked on the engine's own inputs."""

    def __init__(self):
        self.calls = []  # (layer, which, input clone); which = PROJ_* or "attend"

    def project(self, layer, which, in_ptr, out_ptr, rows, stream):
        n_in = _n_in(which)
        with torch.cuda.stream(torch.cuda.ExternalStream(stream)):
            self.calls.append((layer, which, _view(in_ptr, rows * n_in).view(rows, n_in).clone()))
        return project(layer, which, in_ptr, out_ptr, rows, stream)

    def attend(self, layer, q_ptr, kc, vc, kv_dtype, pos_ptr, n_tok, max_seq, out_ptr, stream):
        n = NQ * n_tok * HD
        with torch.cuda.stream(torch.cuda.ExternalStream(stream)):
            self.calls.append((layer, "attend", _view(q_ptr, n).view(NQ, n_tok, HD).clone()))
        return attend(layer, q_ptr, kc, vc, kv_dtype, pos_ptr, n_tok, max_seq, out_ptr, stream)


def _rel_ok(got, want, what):
    """RMSNorm outputs: <= 1e-5 relative per element (the sum's order differs from the serial fold)."""
    err = np.abs(got - want)
    assert np.all(err <= 1e-5 * np.abs(want)), f"{what}: max rel {float((err / np.maximum(np.abs(want), 1e-30)).max())}"


def _teacher_forced(orc, model, layout, steps, max_seq, max_chunk, what):
    """Run `steps` (lists of ids: one id = forward_token, more = forward_chunk) through an engine
    whose stand-ins record what each op received, and check every op of every layer on those
    inputs: the residual stream x is rebuilt from the records with the same f32 adds (exact);
    RMSNorm (input, post-attention, final) to 1e-5 relative, bias + RoPE of q (the attention input)
    and of k with the v rows (the caches) and SwiGLU bit for bit, so no op's tolerance compounds
    over the layers. Reference sequence: wgpu_engine.rs:362-629."""
    table, layers, final = model
    tab = to_np(table)
    lw = [{k: (None if v is None else widen(v, orc)) for k, v in Lw.items()} for Lw in layers]
    fin = to_np(final)
    rec = _Recorder()
    cfg = L.EngineConfig(H, NQ, NKV, HD, INTER, LAYERS, max_seq, max_chunk, EPS, THETA, layout, L.F16, L.F16)
    eng = Engine(cfg, table, L.F32, VOCAB, layers, final, rec.project, rec.attend)
    if layout == L.ROPE_NEOX:
        rope = lambda x, pos: orc.apply_rope(x, pos, THETA)
    else:  # interleaved pairs (the GGUF q/k layout), full rotary dimension
        rope = lambda x, pos: orc.apply_rope_partial_scaled(x, pos, THETA, HD, 1.0, True)
    proj = lambda x, n_out: (0.5 * np.tile(x, (1, -(-n_out // x.shape[1])))[:, :n_out]).astype(np.float32)
    caches = [(np.zeros((NKV, max_seq, HD), np.uint16), np.zeros((NKV, max_seq, HD), np.uint16))
              for _ in range(LAYERS)]
    pos0 = 0
    for si, ids in enumerate(steps):
        rec.calls.clear()
        out = to_np(eng.forward_chunk(ids) if len(ids) > 1 else eng.forward_token(ids[0]))
        torch.cuda.synchronize()
        T = len(ids)
        pos = np.arange(pos0, pos0 + T)
        got = {}
        for layer, which, t in rec.calls:
            got[(layer, which)] = to_np(t)
        print(f"case {what} layout {layout} step {si} positions {pos0}..{pos0 + T - 1}", flush=True)
        x = orc.embed_tokens(tab.reshape(-1).view(np.uint8), L.F32, VOCAB, H, np.array(ids, np.uint32)).reshape(T, H)
        down = None
        for l in range(LAYERS):
            if l > 0:
                x = orc.add(x, down)
            h1 = got[(l, L.PROJ_Q)]
            _rel_ok(h1, orc.rms_norm(x, lw[l]["input_ln"], EPS), f"step {si} layer {l} input norm")
            q = orc.add_bias_last_dim(proj(h1, NQ * HD), lw[l]["bq"])
            k = orc.add_bias_last_dim(proj(got[(l, L.PROJ_K)], NKV * HD), lw[l]["bk"])
            v = orc.add_bias_last_dim(proj(got[(l, L.PROJ_V)], NKV * HD), lw[l]["bv"])
            qr = rope(np.ascontiguousarray(q.reshape(T, NQ, HD).transpose(1, 0, 2)[None]), pos)[0]
            kr = rope(np.ascontiguousarray(k.reshape(T, NKV, HD).transpose(1, 0, 2)[None]), pos)[0]
            assert np.array_equal(got[(l, "attend")].view(np.uint32), qr.view(np.uint32)), f"step {si} layer {l} rope q"
            orc.kv_append(kr, caches[l][0], L.F16, NKV, T, HD, max_seq, pos0)
            orc.kv_append(np.ascontiguousarray(v.reshape(T, NKV, HD).transpose(1, 0, 2)), caches[l][1], L.F16, NKV, T,
                          HD, max_seq, pos0)
            attn = got[(l, L.PROJ_O)]
            assert np.array_equal(attn.view(np.uint32), qr.transpose(1, 0, 2).reshape(T, NQ * HD).view(np.uint32))
            x = orc.add(x, proj(attn, H))
            h2 = got[(l, L.PROJ_GATE)]
            _rel_ok(h2, orc.rms_norm(x, lw[l]["post_ln"], EPS), f"step {si} layer {l} post-attention norm")
            act = got[(l, L.PROJ_DOWN)]
            assert np.array_equal(act.view(np.uint32), orc.swiglu(proj(h2, INTER), proj(h2, INTER)).view(np.uint32)), \
                f"step {si} layer {l} swiglu"
            down = proj(act, H)
        _rel_ok(out, orc.rms_norm(orc.add(x[-1:], down[-1:]), fin, EPS)[0], f"step {si} final norm")
        pos0 += T
    for l in range(LAYERS):
        for j, which in enumerate("kv"):
            g = to_np(eng.cache(l, which)).view(np.uint16).reshape(NKV, max_seq, HD)
            assert np.array_equal(g, caches[l][j]), f"layer {l} {which} cache"
    eng.close()


@pytest.mark.parametrize("layout", [L.ROPE_NEOX, L.ROPE_INTERLEAVED], ids=["neox", "interleaved"])
def test_engine_each_op_on_its_own_inputs(dev, orc, model, layout):
    """Teacher-forced parity of a prompt chunk and decode steps."""
    _teacher_forced(orc, model, layout, [PROMPT] + [[t] for t in DECODE], MAX_SEQ, MAX_CHUNK, "engine teacher-forced")


def _growth_steps():
    """Chunks before, across and after each fill boundary of the angle table (256, 512, the cap at
    max_seq = 600), single tokens between them, and a last chunk ending at max_seq."""
    rng = np.random.default_rng(7)
    ids = lambda n: [int(t) for t in rng.integers(0, VOCAB, n)]
    steps = [ids(16) for _ in range(15)]                 # 0 .. 239: the first fill covers 256 rows
    steps += [[t] for t in ids(5)]                        # 240 .. 244 one token at a time
    steps += [ids(16)]                                    # 245 .. 260: across 256, the table grows to 512
    steps += [ids(16) for _ in range(15)]                 # 261 .. 500
    steps += [ids(3), ids(16)]                            # 501 .. 503, then 504 .. 519 across 512: to 600
    steps += [[t] for t in ids(50)]                       # 520 .. 569
    steps += [ids(14), ids(16)]                           # 570 .. 583, 584 .. 599: ends at max_seq
    assert sum(len(s) for s in steps) == 600
    return steps


def test_engine_chunks_across_angle_table_growth(dev, orc, model):
    """A chunk's RoPE angles are the rows of the engine's per-position table that its positions name,
    filled from the host as positions are first reached (256 rows, then doubling up to max_seq);
    a one-token step's angles are staged per step. Every step teacher-forced."""
    _teacher_forced(orc, model, L.ROPE_NEOX, _growth_steps(), 600, 16, "engine angle table")


def test_graph_run_equals_eager_across_angle_table_growth(dev, model):
    """Graph mode (replayed single tokens between eager chunks that grow the angle table) is bit
    for bit the eager run."""
    table, layers, final = model
    cfg = L.EngineConfig(H, NQ, NKV, HD, INTER, LAYERS, 600, 16, EPS, THETA, L.ROPE_NEOX, L.F16, L.F16)
    steps = _growth_steps()
    runs = []
    for graph in (False, True):
        eng = Engine(cfg, table, L.F32, VOCAB, layers, final, project, attend)
        runs.append((eng, _run(eng, graph, steps)))
    print("case engine graph chunks vs eager, growth run", flush=True)
    (eager, e_out), (graph, g_out) = runs
    for i, (a, b) in enumerate(zip(e_out, g_out)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {i}"
    for l in range(LAYERS):
        for w in "kv":
            assert torch.equal(eager.cache(l, w), graph.cache(l, w)), f"layer {l} {w} cache"
    eager.close()
    graph.close()
