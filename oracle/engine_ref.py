"""Oracle: one-token-at-a-time decoding with a key cache (batch 1).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Restates engine.py:14-177 of the reference, generalised
to the (leaf, arity) tree, and optionally run in bfloat16 activations (the same op chain on bf16 tensors)
for the bf16 decode configurations.  Also used as the CPU baseline of bench.py (one sequence).
"""
import math

import torch
import torch.nn.functional as F

from .attn_ref import dedupe, dedupe_fast, local_block, static_keys
from .seg_ref import (Geometry, dot_canonical, finish, gate_apply, gather_nodes, index_log, injected, neighbor_pass,
                      rank_canonical, tree_pass)


def _ln(x, w):
    return F.layer_norm(x, (x.shape[-1],), w, None, 1e-5)


class SegStateRef:
    """Per-layer decode cache (engine.py:18-71): K and V rows (float32), node sums at every binary level
    0..l_J (a node is formed, as the sum of its two children, when its last position arrives), the leaves
    each earlier query found (for neighbour borrowing) and the running key sum."""

    def __init__(self, cfg, Tcap, H, dh, canon=False):
        self.cfg, self.Tcap, self.H, self.dh = cfg, Tcap, H, dh
        self.canon = canon   # the gate's canonical log and quantile (seg_ref.index_log, quantile_canon)
        self.geom = Geometry(Tcap, getattr(cfg, 'leaf', 2), getattr(cfg, 'arity', 2))
        self.Ltop = self.geom.blevels[-1] if self.geom.J >= 0 else 0
        self.Lm = self.Ltop
        self.K = torch.zeros(1, H, Tcap, dh)
        self.V = torch.zeros(1, H, Tcap, dh)
        self.raw = [torch.zeros(1, H, Tcap >> l, dh) for l in range(self.Ltop + 1)]
        self.lg = [torch.zeros(1, H, Tcap >> l, dh) for l in range(self.Ltop + 1)] if cfg.gate else None
        NS = cfg.nb_store
        self.st_leaf = torch.zeros(1, H, Tcap, NS, dtype=torch.long)
        self.st_score = torch.zeros(1, H, Tcap, NS)
        self.st_ok = torch.zeros(1, H, Tcap, NS, dtype=torch.bool)
        self.ksum = torch.zeros(1, H, dh)

    def getU(self, l, cand):
        """Node vectors of `cand` at binary level l, gated at l >= gate_min_level (engine.py:35-39)."""
        U = gather_nodes(self.raw[l], cand)
        if self.cfg.gate and l >= getattr(self.cfg, 'gate_min_level', 0):
            U = gate_apply(U, gather_nodes(self.lg[l], cand), float(1 << l), self.cfg.gate_q, self.canon)
        return U

    def add(self, t, k, v):
        """Store position t (k, v: (1,H,dh)); form every node whose last child just completed (engine.py:41-55)."""
        self.K[:, :, t] = k.float()
        self.V[:, :, t] = v.float()
        kidx = torch.zeros_like(k.float()) if t == 0 else k.float()
        self.raw[0][:, :, t] = kidx
        if self.lg is not None:
            self.lg[0][:, :, t] = index_log(kidx, self.canon)
        for l in range(1, self.Ltop + 1):
            if (t + 1) % (1 << l):
                break
            n = t >> l
            self.raw[l][:, :, n] = self.raw[l - 1][:, :, 2 * n] + self.raw[l - 1][:, :, 2 * n + 1]
            if self.lg is not None:
                self.lg[l][:, :, n] = self.lg[l - 1][:, :, 2 * n] + self.lg[l - 1][:, :, 2 * n + 1]
        self.ksum = self.ksum + k.float()

    def fill(self, K, V):
        """Load a whole context at once (engine.py:57-71)."""
        H, dh = self.H, self.dh
        self.K, self.V = K.float().clone(), V.float().clone()
        kidx = self.K.clone()
        kidx[:, :, 0] = 0
        self.raw[0] = kidx
        lg = index_log(kidx, self.canon) if self.lg is not None else None
        if lg is not None:
            self.lg[0] = lg
        for l in range(1, self.Ltop + 1):
            self.raw[l] = self.raw[l - 1].reshape(1, H, self.Tcap >> l, 2, dh).sum(3)
            if lg is not None:
                self.lg[l] = self.lg[l - 1].reshape(1, H, self.Tcap >> l, 2, dh).sum(3)
        self.ksum = self.K.sum(2)


def descend(state, q, t, mode):
    """Beam descent of one query over the cache: the literal reference pass at (2, 2) in faithful mode,
    otherwise the generalised pass in the requested mode."""
    geom = state.geom
    tq = torch.tensor([t])
    if geom.J < 0:
        z = torch.zeros(1, state.H, 1, 0)
        return z.long(), z.bool(), z
    if mode == 'faithful' and geom.leaf == 2 and geom.arity == 2:
        return tree_pass(q, state.getU, tq, geom.blevels[-1], state.cfg.wmax)
    a = geom.arity
    H = state.H
    ids = vld = sct = None
    for j in range(geom.J, -1, -1):
        l = geom.blevels[j]
        inj, injv = injected(tq, l, a)
        inj = inj.view(1, 1, 1, a - 1).expand(1, H, 1, a - 1)
        injv = injv.view(1, 1, 1, a - 1).expand(1, H, 1, a - 1)
        if ids is None:
            cand, cv = inj, injv
        else:
            cand = torch.cat([a * ids + c for c in range(a)] + [inj], -1)
            cv = torch.cat([vld] * a + [injv], -1)
        U = state.getU(l, cand.clamp(0, state.raw[l].shape[2] - 1))
        w = min(state.cfg.wmax, cand.shape[-1])
        if mode == 'faithful':
            sc = ((q.unsqueeze(3) * U).sum(-1) / float(1 << l)).masked_fill(~cv, float('-inf'))
            sct, order = sc.topk(w, dim=-1)
        else:
            sc = (dot_canonical(q, U) * (1.0 / float(1 << l))).masked_fill(~cv, float('-inf'))
            order = rank_canonical(sc, cand, cv, w)
            sct = sc.gather(-1, order)
        ids, vld = cand.gather(-1, order), cv.gather(-1, order)
    return ids, vld, sct


def budget(state, pw, q, t):
    """Leaf budget lhat (1,H,1): the fixed beam, or the budget head's class (engine.py:89-96)."""
    cfg, H = state.cfg, state.H
    if cfg.beam_mode == 'pred':
        feats = [q, torch.log(q.norm(dim=-1, keepdim=True) + 1e-6), torch.eye(H).view(1, H, 1, H)]
        if cfg.global_pool:
            feats.append((state.ksum / max(t, 1)).unsqueeze(2))
        h = F.relu(F.linear(torch.cat(feats, -1), pw['w1'].float(), pw['b1'].float()))
        return pw['classes'][F.linear(h, pw['w2'].float(), pw['b2'].float()).argmax(-1)]
    return torch.full((1, H, 1), cfg.beam, dtype=torch.long)


@torch.no_grad()
def seg_attend_ref(state, pw, q, k, v, t, update=True, mode='faithful', want_sel=False, sort_dedupe=False):
    """One decode step of one layer (engine.py:84-120): budget, descent over the cache (positions < t),
    neighbour pass over the stored leaves, budget split, store this query's leaves and add position t,
    candidate assembly with the static keys (and the own leaf block when leaf > 2), K x K de-duplication,
    softmax attention in fp32.  q, k, v: (1,H,1,dh).  Returns (out (1,H,1,dh) fp32, mean keys per head)."""
    cfg, H, dh = state.cfg, state.H, state.dh
    leaf = state.geom.leaf
    q = q.float()
    lhat = budget(state, pw, q, t)
    tq = torch.tensor([t])
    ids, vld, sct = descend(state, q, t, mode)
    NS = cfg.nb_store
    dot = (lambda a, b: (a.unsqueeze(3) * b).sum(-1)) if mode == 'faithful' else dot_canonical
    if state.geom.J >= 0:
        getU1 = lambda c: state.getU(state.geom.blevels[0], c)
        nid, match, nL = neighbor_pass(q, getU1, state.st_leaf, state.st_score, state.st_ok, tq, cfg, leaf,
                                       lambda a, b: dot(a, b))
    else:
        Wn = cfg.nb_window
        nid = torch.zeros(1, H, 1, Wn * NS, dtype=torch.long)
        match = torch.zeros(1, H, 1, Wn * NS, dtype=torch.bool)
        nL = torch.zeros(1, H, 1, dtype=torch.long)
    sel = finish(ids, vld, nid, match, nL, lhat, cfg, leaf)
    if update:
        n = min(NS, ids.shape[-1])
        state.st_leaf[:, :, t, :n] = ids[:, :, 0, :n]
        state.st_score[:, :, t, :n] = sct[:, :, 0, :n]
        state.st_ok[:, :, t, :n] = vld[:, :, 0, :n]
        state.add(t, k[:, :, 0], v[:, :, 0])
    wl = ids.shape[-1]
    parts = [static_keys(tq, cfg.local)]
    if leaf > 2:
        parts.append(local_block(tq, leaf))
    extra = torch.cat(parts, 1).view(1, 1, 1, -1).expand(1, H, 1, -1)
    cand = torch.cat([sel['tree_pos'], sel['nb_pos'], extra], -1)
    used = sel['leaf_ok'] & (torch.arange(wl) < sel['n_tree'].unsqueeze(-1))
    tv = torch.cat([used] * leaf, -1) & (sel['tree_pos'] >= 0)
    # the K x K comparison of engine.py:114, or the equal sort-based form (fastseg.py:227-234) for long lists
    keep = (dedupe_fast if sort_dedupe else dedupe)(cand, torch.cat([tv, sel['nb_pos'] >= 0, extra >= 0], -1))
    idx = cand.clamp(min=0)
    kg, vg = gather_nodes(state.K, idx), gather_nodes(state.V, idx)
    s = (q.unsqueeze(3) * kg).sum(-1) * (1.0 / math.sqrt(dh))
    w = torch.softmax(s.masked_fill(~keep, float('-inf')), -1)
    out = (w.unsqueeze(-1) * vg).sum(3)
    kr = keep.float().sum(-1).mean().item()
    if want_sel:
        return out, kr, dict(ids=ids, vld=vld, sct=sct, used=used, cand=cand, keep=keep)
    return out, kr


def weights_from_ours(sd, cfg):
    """Engine weight dict from a model state_dict (engine.py:123-134)."""
    W = dict(wte=sd['wte.weight'], wpe=sd['wpe.weight'], ln_f=sd['ln_f.weight'], layers=[])
    for i in range(cfg.n_layer):
        p = 'blocks.%d.' % i
        L = dict(ln1=sd[p + 'ln1.weight'], c_attn=sd[p + 'attn.c_attn.weight'], c_proj=sd[p + 'attn.c_proj.weight'],
                 ln2=sd[p + 'ln2.weight'], c_fc=sd[p + 'mlp.c_fc.weight'], c_mlp=sd[p + 'mlp.c_proj.weight'])
        if cfg.beam_mode == 'pred':
            L['pw'] = dict(w1=sd[p + 'attn.pred.0.weight'], b1=sd[p + 'attn.pred.0.bias'],
                           w2=sd[p + 'attn.pred.2.weight'], b2=sd[p + 'attn.pred.2.bias'],
                           classes=torch.tensor(list(cfg.beam_classes)))
        W['layers'].append(L)
    return W


def linear_f32_round(x, w):
    """A linear layer as a float32 product of the operands rounded once to x's dtype: for bf16 operands the
    same real quantity as F.linear accumulated in another order.  A DecoderRef built with it measures the
    rounding noise floor of a bf16 op chain against one built with F.linear."""
    return (x.float() @ w.float().t()).to(x.dtype)


class DecoderRef:
    """Token-by-token decoder (engine.py:149-177).  act_dtype=torch.bfloat16 runs the same op chain on
    bf16 activations and weights (the bf16 decode configurations); selection and attention stay fp32."""

    def __init__(self, W, n_layer, n_head, n_embd, Tcap, mode='seg', cfg=None, act_dtype=torch.float32,
                 sel_mode='faithful', linear=None, sort_dedupe=False):
        self.W, self.nl, self.H, self.C, self.Tcap = W, n_layer, n_head, n_embd, Tcap
        self.dh, self.mode, self.cfg = n_embd // n_head, mode, cfg
        self.dt = act_dtype
        self.sel_mode = sel_mode
        # the matrix product of every linear layer (F.linear; another float32-accumulating product rounded to
        # the activation dtype gives an equally valid bf16 result, which measures the rounding noise floor)
        self.lin = linear or F.linear
        self.sort_dedupe = sort_dedupe
        self.reset()

    def reset(self):
        self.states = [SegStateRef(self.cfg, self.Tcap, self.H, self.dh, canon=self.sel_mode == 'canonical')
                       for _ in range(self.nl)]

    @torch.no_grad()
    def step(self, tok, t, want_sel=False, probe=None):
        """Feed token `tok` at position t -> (logits (V,) fp32, mean keys read per head and layer).
        probe(i, values), when given, sees every layer's intermediate tensors (x_in, q, k, v, out, x_mid, h,
        x_out) and finally probe('final', dict(x, logits)) -- for comparing another implementation op by op."""
        W, H, C, dh, dt = self.W, self.H, self.C, self.dh, self.dt
        x = (W['wte'][tok].to(dt) + W['wpe'][t].to(dt)).view(1, 1, C)
        keys = 0.0
        sels = []
        for i, L in enumerate(W['layers']):
            x_in = x
            q, k, v = self.lin(_ln(x, L['ln1'].to(dt)), L['c_attn'].to(dt)).split(C, -1)
            q, k, v = [a.view(1, 1, H, dh).transpose(1, 2) for a in (q, k, v)]
            res = seg_attend_ref(self.states[i], L.get('pw'), q, k, v, t, mode=self.sel_mode,
                                 want_sel=want_sel or probe is not None, sort_dedupe=self.sort_dedupe)
            out, kr = res[0], res[1]
            if want_sel:
                sels.append(res[2])
            keys += kr
            x = x + self.lin(out.to(dt).transpose(1, 2).reshape(1, 1, C), L['c_proj'].to(dt))
            x_mid = x
            h = F.gelu(self.lin(_ln(x, L['ln2'].to(dt)), L['c_fc'].to(dt)))
            x = x + self.lin(h, L['c_mlp'].to(dt))
            if probe is not None:
                probe(i, dict(x_in=x_in, q=q, k=k, v=v, out=out, x_mid=x_mid, h=h, x_out=x, sel=res[2]))
        logits = self.lin(_ln(x, W['ln_f'].to(dt)), W['wte'].to(dt))[0, 0].float()
        if probe is not None:
            probe('final', dict(x=x, logits=logits))
        if want_sel:
            return logits, keys / self.nl, sels
        return logits, keys / self.nl
