"""Paged decode caches (a page = the K and V rows of one leaf block of one (sequence, head)) against the
contiguous layout: every kernel that reads or writes the cache, and the decoder, give bit-identical results,
with pages handed out in a scrambled order.  GPU only."""
import math

import pytest
import torch

from oracle import seg_ref as S
from treeattn_amd import kernels as K
from treeattn_amd.config import Config
from treeattn_amd.engine import Decoder, PagePool, weights_from_ours
from treeattn_amd.model import GPT

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def rnd(*shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def scrambled_pages(K_, V_, leaf, spare=7, seed=0):
    """A PagedCache holding the contiguous cache K_, V_ (B,H,T,D) in randomly ordered pages (plus spare ones)."""
    B, H, T, D = K_.shape
    nb = T // leaf
    P = B * H * nb + spare
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(P, generator=g)[:B * H * nb].to(torch.int32)
    table = perm.view(B, H, nb).contiguous().to(DEV)
    pool = torch.zeros(P, 2, leaf, D, dtype=K_.dtype, device=DEV)
    pg = table.long().reshape(-1)
    pool[pg, 0] = K_.reshape(B, H, nb, leaf, D).reshape(-1, leaf, D)
    pool[pg, 1] = V_.reshape(B, H, nb, leaf, D).reshape(-1, leaf, D)
    return K.PagedCache(pool, table, T)


@pytest.mark.parametrize('dtype,D,leaf,arity', [(torch.float32, 64, 8, 2), (torch.bfloat16, 64, 64, 2),
                                                (torch.bfloat16, 128, 16, 4)])
def test_kv_append_paged_equals_contiguous(dtype, D, leaf, arity):
    B, H, Tcap = 2, 3, 512
    shape = K.TreeShape(Tcap, leaf, arity)
    Kd = torch.zeros(B, H, Tcap, D, device=DEV, dtype=dtype)
    Vd = torch.zeros_like(Kd)
    pc = scrambled_pages(Kd, Vd, leaf)
    lv_d = [t.zero_() for t in shape.alloc_levels(B, H, D, DEV)]
    lv_p = [t.zero_() for t in shape.alloc_levels(B, H, D, DEV)]
    kk, vv = rnd(Tcap, B, H, D, seed=1, dtype=dtype).to(DEV), rnd(Tcap, B, H, D, seed=2, dtype=dtype).to(DEV)
    tpos = torch.zeros(B, dtype=torch.int32, device=DEV)
    for t in range(Tcap):
        tpos.fill_(t)
        K.kv_append(kk[t], vv[t], Kd, Vd, tpos, lv_d, leaf, arity)
        K.kv_append(kk[t], vv[t], pc, None, tpos, lv_p, leaf, arity)
    for b in range(B):
        kb, vb = pc.dense(b)
        assert torch.equal(kb, Kd[b:b + 1]) and torch.equal(vb, Vd[b:b + 1])
    for a, c in zip(lv_d, lv_p):
        assert torch.equal(a, c)


def _selection(q, k, tq, leaf, wmax):
    T = k.shape[2]
    geom = S.Geometry(T, leaf, 2)
    ids, vld, _ = S.tree_pass_general(q.float().cpu(), S.pyramid(S.index_keys(k.cpu()), geom), tq, geom, wmax,
                                      'canonical')
    return torch.where(vld, ids, -1).to(torch.int32).to(DEV), vld.to(torch.uint8).to(DEV)


@pytest.mark.parametrize('nsplit', [4, 16])
def test_seg_attn_paged_equals_contiguous(nsplit):
    B, H, T, D, leaf, wmax = 2, 3, 2048, 64, 32, 8
    q, k, v = [rnd(B, H, T, D, seed=s, dtype=torch.bfloat16) for s in (3, 4, 5)]
    nq = 24
    tq = torch.arange(T - nq, T)
    qs = q[:, :, T - nq:].contiguous().to(DEV)
    ids, vld = _selection(qs, k, tq, leaf, wmax)
    kd, vd = k.to(DEV), v.to(DEV)
    pc = scrambled_pages(kd, vd, leaf, seed=1)
    args = (tq.to(torch.int32).to(DEV), ids, vld, None, leaf, 3, 1 / math.sqrt(D))
    od, ld, kyd = K.seg_attn(qs, kd, vd, *args, lse=torch.empty(B, H, nq, device=DEV),
                             keys=torch.empty(B, H, nq, device=DEV), nsplit=nsplit)
    op, lp, kyp = K.seg_attn(qs, pc, None, *args, lse=torch.empty(B, H, nq, device=DEV),
                             keys=torch.empty(B, H, nq, device=DEV), nsplit=nsplit)
    assert torch.equal(od, op) and torch.equal(ld, lp) and torch.equal(kyd, kyp)
    # one wavefront per query over pages (the contiguous prefill shape runs on the matrix cores instead, which
    # round the probabilities to bf16: within the bf16 bar)
    o1, _, k1 = K.seg_attn(qs, pc, None, *args, keys=torch.empty(B, H, nq, device=DEV), nsplit=1)
    assert torch.equal(k1, kyd) and (o1.float() - od.float()).abs().max().item() < 2e-2


def test_sparse_attn_candidates_paged_equals_contiguous():
    """The candidate-list attention (neighbour-borrowing decode) over a paged cache."""
    B, H, T, D, leaf = 1, 2, 1024, 64, 16
    q = rnd(B, H, 4, D, seed=6).to(DEV)
    k, v = rnd(B, H, T, D, seed=7).to(DEV), rnd(B, H, T, D, seed=8).to(DEV)
    g = torch.Generator().manual_seed(9)
    cand = torch.randint(-1, T, (B, H, 4, 70), generator=g).to(DEV)
    pc = scrambled_pages(k, v, leaf, seed=2)
    od, ld = K.sparse_attn_fwd(q, k, v, cand, 0.125)
    op, lp = K.sparse_attn_fwd(q, pc, None, cand, 0.125)
    assert torch.equal(od, op) and torch.equal(ld, lp)


@pytest.mark.parametrize('D', [64, 128])
def test_seg_attend_paged_equals_contiguous(D):
    """The one-launch layer attention (append + descent + attention) writes and reads the same rows."""
    B, H, Tcap, leaf, wmax = 3, 4, 1024, 32, 8
    shape = K.TreeShape(Tcap, leaf, 2)
    T0 = 700
    k0, v0 = rnd(B, H, Tcap, D, seed=10, dtype=torch.bfloat16), rnd(B, H, Tcap, D, seed=11, dtype=torch.bfloat16)
    k0[:, :, T0:] = 0
    v0[:, :, T0:] = 0
    Kd, Vd = k0.to(DEV), v0.to(DEV)
    pc = scrambled_pages(Kd, Vd, leaf, seed=3)
    lv_d = K.level_sums(Kd, shape.blevels, t_end=T0)
    lv_p = [t.clone() for t in lv_d]
    wl = shape.leaf_width(wmax)
    n_tree = torch.full((B, H, 1), wmax, dtype=torch.int32, device=DEV)
    for s in range(40):
        t = T0 + s
        q = rnd(B, H, 1, D, seed=100 + s, dtype=torch.bfloat16).to(DEV)
        kn = rnd(B, H, D, seed=200 + s, dtype=torch.bfloat16).to(DEV)
        vn = rnd(B, H, D, seed=300 + s, dtype=torch.bfloat16).to(DEV)
        tpos = torch.full((B,), t, dtype=torch.int32, device=DEV)
        outs = []
        for Kc, Vc, lv in ((Kd, Vd, lv_d), (pc, None, lv_p)):
            sel = (torch.empty(B, H, 1, wl, dtype=torch.int32, device=DEV),
                   torch.empty(B, H, 1, wl, dtype=torch.uint8, device=DEV), torch.empty(B, H, 1, wl, device=DEV))
            out = torch.empty(B, H, 1, D, dtype=torch.bfloat16, device=DEV)
            keys = torch.empty(B, H, 1, device=DEV)
            K.seg_attend(q, lv, tpos, shape, wmax, kn, vn, Kc, Vc, n_tree, 3, 1 / math.sqrt(D), sel, out, keys=keys)
            outs.append((out, keys) + sel)
        for a, c in zip(*outs):
            assert torch.equal(a, c), s
    for a, c in zip(lv_d, lv_p):
        assert torch.equal(a, c)


def test_append_without_page_writes_nothing():
    """A row whose leaf block has no page (-1) is neither stored nor summed into a node."""
    B, H, D, leaf, Tcap = 1, 2, 64, 8, 64
    shape = K.TreeShape(Tcap, leaf, 2)
    table = torch.full((B, H, Tcap // leaf), -1, dtype=torch.int32, device=DEV)
    table[:, :, 0] = torch.tensor([0, 1], dtype=torch.int32)
    pool = torch.zeros(3, 2, leaf, D, device=DEV)
    pc = K.PagedCache(pool, table, Tcap)
    lv = [t.zero_() for t in shape.alloc_levels(B, H, D, DEV)]
    kn = torch.ones(B, H, D, device=DEV)
    K.kv_append(kn, kn, pc, None, torch.tensor([leaf + leaf - 1], dtype=torch.int32, device=DEV), lv, leaf, 2)
    torch.cuda.synchronize()
    assert pool.abs().sum().item() == 0 and all(t.abs().sum().item() == 0 for t in lv)


@pytest.mark.parametrize('kw', [dict(neighbors=False, leaf=8, wmax=4, beam=4), dict(leaf=4, wmax=4, beam=3),
                                dict(beam_mode='pred', global_pool=True, leaf=8, wmax=8),
                                dict(gate=True, gate_min_level=4, leaf=8, wmax=4, beam=4)])
def test_decoder_paged_equals_contiguous(kw):
    """Prefill, eager steps and replays of a captured step that cross page boundaries (pages handed out a few
    positions ahead): logits, tokens and node sums equal the contiguous decoder's bit for bit; the pool holds
    pages for the positions reached, not for Tcap."""
    cfg = Config(vocab_size=96, seq_len=512, n_layer=2, n_head=2, n_embd=128, attn='seg', **kw)
    torch.manual_seed(13)
    model = GPT(cfg).eval()
    sd = {k: v.to(torch.bfloat16).to(DEV) for k, v in model.state_dict().items()}
    W = weights_from_ours(sd, cfg)
    g = torch.Generator().manual_seed(14)
    idx = torch.randint(0, 96, (3, 40), generator=g).to(DEV)
    a = Decoder(W, 2, 2, 128, 512, 'seg', cfg, DEV, batch=3, paged=False)
    b = Decoder(W, 2, 2, 128, 512, 'seg', cfg, DEV, batch=3, paged=True, max_tokens=160, reserve_ahead=5)
    assert a.pool is None and b.pool is not None and b.pool.P < 3 * 2 * 512 // cfg.leaf
    la, lb = a.prefill(idx), b.prefill(idx)
    assert torch.equal(la, lb)
    tok = la.float().argmax(-1)
    for t in range(40, 52):
        la, _ = a.step(tok, t)
        lb, _ = b.step(tok, t)
        assert torch.equal(la, lb), t
        tok = la.float().argmax(-1)
    a.capture(tok, 52)
    b.capture(tok, 52)
    for r in range(30):
        a.replay()
        b.replay()
        torch.cuda.synchronize()
        assert torch.equal(a.g_logits, b.g_logits), r
        assert torch.equal(a.g_tok, b.g_tok), r
    for sa, sb in zip(a.states, b.states):
        for s in range(3):
            ka, va = sa.dense_kv(s, 82)
            kb, vb = sb.dense_kv(s, 82)
            assert torch.equal(ka, kb) and torch.equal(va, vb)
        for x, y in zip(sa.levels + (sa.lg or []), sb.levels + (sb.lg or [])):
            assert torch.equal(x, y)
        for x, y in zip(sa.score_levels, sb.score_levels):
            assert torch.equal(x, y)
    assert b.pool.nblk[0] * cfg.leaf < 82 + 16
