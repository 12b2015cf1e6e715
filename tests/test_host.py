"""CPU tests of the host side: the C-ABI library loads and exports every entry include/*.h
declares (no compute call without a GPU), the plan (counts, chain rule, truncation, folds), the
packed seeded layout (segments cover each element once, the shared-expert split, stream names),
and the host-side generators against the oracle's."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from oracle import model as M
from fleet import runtime as R
from fleet import graph_plan as G
from fleet import build_graph as B
from fleet import pack_weights as P

ROOT = Path(__file__).resolve().parent.parent


def test_library_exports_every_declared_symbol():
    hdr = (ROOT / "include" / "fleet_mi355x.h").read_text()
    declared = set(re.findall(r"^\s*(?:int|const char\*)\s+(fx_\w+)\(", hdr, re.M))
    assert declared == set(R.EXPORTS), declared ^ set(R.EXPORTS)
    lib = ctypes.CDLL(str(R.LIB_PATH))
    for name in declared:
        assert hasattr(lib, name), name
    assert R.lib().fx_abi_version() == R.FX_ABI_VERSION == 4


def test_stage_struct_size_matches_header():
    assert ctypes.sizeof(R.FxStage) == 208
    # field offsets shared with the C header: src after the 18 int32 fields, pointers 8-aligned
    assert R.FxStage.src.offset == 72 and R.FxStage.w.offset == 104 and R.FxStage.aux.offset == 144


def test_plan_counts_and_chain():
    p = G.build_plan()
    s = G.summary(p)
    # 1 embed + 27 x (qkva, prep, attend, merge, o_proj) + 2 dense + 26 x 4 MoE calls + 2 head
    assert s["ops"] == 1 + 27 * 5 + 2 + 26 * 4 + 2
    assert p.chain_violations() == []
    # defaults: the matrix-core attention takes 32-position splits (one per worker) up to 32 splits;
    # the vector-ALU and single-XCD attentions at most 32 splits (one per worker of an XCD)
    assert (p.attn, p.split, p.n_splits) == ("mfma", 32, 33)
    assert (G.build_plan(attn="valu").split, G.build_plan(attn="valu").n_splits) == (64, 17)
    xc = G.build_plan(attn="xcd")
    assert (xc.attn, xc.split, xc.n_splits) == ("xcd", 64, 17)
    # beyond 4,096 positions about 128 splits (32 positions per 4,096 of the cache)
    assert G.default_splits(16416) == (128, 129)
    assert G.default_splits(4096) == (32, 128)
    assert (G.build_plan(split=32).split, G.build_plan(split=32).n_splits) == (32, 33)
    t = G.build_plan().truncate("L1.o_proj")
    assert t.calls[-1].label == "L1.o_proj"
    assert G.splits_for(32768, n_splits=32) == (1024, 32)
    assert G.splits_for(16416, n_splits=128) == (160, 103)


class _FakeBuf:
    _next = 0x1000

    def __init__(self, shape, dtype):
        self.shape, self.dtype = tuple(shape), dtype
        _FakeBuf._next += 0x100000
        self.ptr = _FakeBuf._next


class _FakeRt:
    def alloc(self, shape, dtype):
        b = _FakeBuf(shape if isinstance(shape, tuple) else (shape,), dtype)
        b.zero = lambda: b
        return b


def _fake_host(plan):
    rt = _FakeRt()
    host = {}
    for name, t in plan.tensors.items():
        host[name] = rt.alloc(t.shape, t.dtype)
    return host


def test_fold_rules():
    p = G.build_plan(layers=3, head=True)
    host = _fake_host(p)
    stages, epi = B.compile_stages(p, host)
    labels = B.compile_stages.labels
    ops = [s.op for s in stages]
    n = len(stages)
    # embed folded into L0.qkva, combines folded into their w2, argmax as the epilogue
    assert stages[0].op == R.FX_OP_GEMV and stages[0].in_kind == R.FX_IN_EMBED
    assert not any("combine" in l for l in labels)
    assert [e.op for e in epi] == [R.FX_OP_ARGMAX]
    assert n == 7 + 2 * 7 + 1            # layer 0: 7 stages, MoE layers 7 each (router in w13), head 1
    # packet sources: the embed's amax is the previous iteration's head; everything else the stage
    # that last wrote the tensor
    assert stages[0].src[1] == -1 and labels[-1] == "head.lm_head"
    assert epi[0].src[0] == -1
    for i, st in enumerate(stages):
        if st.op == R.FX_OP_MLA_PREP:
            assert labels[st.src[0]].endswith(".qkva") or labels[st.src[0]].endswith(".qkva+embed")
        if st.op == R.FX_OP_MLA_ATTEND:
            assert ops[st.src[0]] == R.FX_OP_MLA_PREP and st.src[0] == i - 1
        if st.op == R.FX_OP_MOE_W13:
            assert st.flags & R.FX_F_ROUTER and labels[i].endswith(".w13+router") and st.res
        if st.op == R.FX_OP_MOE_W2:
            assert ops[st.src[0]] == R.FX_OP_MOE_W13 and st.src[1] == st.src[0]
            assert labels[st.src[2]].endswith(".o_proj") and st.out == host["x_res"].ptr and st.res == host["x_mid"].ptr
    # layer 0's o_proj takes the embedding row as its residual; later o_projs the x_res packets
    o0 = stages[labels.index("L0.o_proj")]
    assert o0.flags & R.FX_F_RES_EMBED and not o0.flags & R.FX_F_RESIDUAL
    o1 = stages[labels.index("L1.o_proj")]
    assert o1.flags & R.FX_F_RESIDUAL and o1.res == host["x_res"].ptr and o1.out == host["x_mid"].ptr
    assert ops[o1.src[2]] == R.FX_OP_GEMV and labels[o1.src[2]] == "L0.down"
    # a plan truncated after a w2 keeps its combine (the same stage)
    t = G.build_plan(layers=3, head=False).truncate("L1.w2")
    assert t.calls[-1].label == "L1.combine"
    st, _ = B.compile_stages(t, _fake_host(t))
    assert st[-1].op == R.FX_OP_MOE_W2 and st[0].src[1] == -1
    # a plan truncated after a router runs it alone
    t = G.build_plan(layers=3, head=False).truncate("L1.router")
    st, _ = B.compile_stages(t, _fake_host(t))
    assert st[-1].op == R.FX_OP_MOE_ROUTER


def test_seeded_layout_segments_cover_each_element_once():
    d = P.Dims(H=2048, NH=16, D_N=128, D_R=64, D_V=128, D_C=512, V=512, L=2, I_DENSE=64, I_MOE=64, E=6, TOPK=6,
               N_SHARED=2)
    for key, pt in P.seeded_layout(d).items():
        if pt.init == "ones":
            continue
        cover = np.zeros(pt.numel, np.int32)
        for s in pt.init:
            for r in range(s.rows):
                o = s.dst_offset + r * s.dst_stride
                cover[o:o + s.row_len] += 1
        assert (cover == 1).all(), key


def test_shared_expert_halves_equal_the_fused_shared_mlp():
    """pack_moe (the reference's pack_weights.py:187-210): experts E and E+1 are the two halves of the
    shared MLP, so sum over both halves of down(silu(gate) * up) equals the shared MLP."""
    d = P.Dims(H=2048, NH=16, D_N=128, D_R=64, D_V=128, D_C=512, V=512, L=2, I_DENSE=64, I_MOE=64, E=6, TOPK=6,
               N_SHARED=2)
    lay = P.seeded_layout(d)
    gen = lambda seed, stream, n, scale, offset: O.gen_normal_bf16(seed, stream, n, scale, offset=offset)
    W13 = P.materialize(lay["W13_1"], 3, gen).astype(np.uint16)
    W2 = P.materialize(lay["W2_1"], 3, gen)
    name = "model.layers.1.mlp.shared_experts."
    I, H = d.I_MOE, d.H
    sg = O.gen_normal_bf16(3, P.fnv1a32(name + "gate_proj.weight"), 2 * I * H, 0.02).reshape(2 * I, H)
    sd = O.gen_normal_bf16(3, P.fnv1a32(name + "down_proj.weight"), H * 2 * I, 0.02).reshape(H, 2 * I)
    assert np.array_equal(W13[6, :I], sg[:I]) and np.array_equal(W13[7, :I], sg[I:])
    assert np.array_equal(W2[6], sd[:, :I]) and np.array_equal(W2[7], sd[:, I:])


def test_stream_names_unique():
    names = ["model.embed_tokens.weight", "lm_head.weight"]
    for l in range(27):
        names += P.layer_names(P.REAL_DIMS, l)
    ids = [P.fnv1a32(n) for n in names]
    assert len(set(ids)) == len(ids)


def test_host_philox_and_tables_match_oracle():
    blocks = np.arange(0, 50, dtype=np.uint64)
    mine = P.philox4x32(99, blocks, 1234)
    for b in (0, 7, 49):
        c = np.array([b, 0, 1234, 0x5EED], np.uint32)
        k = np.array([99, 0], np.uint32)
        assert np.array_equal(mine[b], O.philox4x32_raw(c, k))
    assert np.array_equal(P.prompt_ids(5, 1000, 102400), O.gen_tokens(5, P.fnv1a32("prompt"), 1000, 102400))
    c1, s1 = P.rope_tables(1100)
    c2, s2 = M.rope_tables(1100)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2)


def test_bytes_per_token_matches_the_hand_count():
    # weights read once per token (4,902,874,112 B with the norms) + 27 x 1,152 B of latent cache per
    # attended position: 4,934,724,608 B at the first token (ctx 1024), 5,412,482,048 B at ctx 16,384
    assert P.bytes_per_token(P.REAL_DIMS, 1024) == 4_934_724_608
    assert P.bytes_per_token(P.REAL_DIMS, 16384) == 5_412_482_048
    assert P.packed_bytes(P.REAL_DIMS) == 31_412_968_448
