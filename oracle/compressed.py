"""Compressed-memory mixers CSA and HCA (test infrastructure only: imported by
tests, ``__graft_entry__.smoke`` and bench.py's CPU baseline, never by the
product path).

Restates model/layers/csa.py:16-259, model/layers/hca.py:15-193 and the causal
temporal compressor of model/layers/compressed_attention.py:82-211.  Both
mixers are one computation with different shapes:

  * index heads: H heads of width Dh for queries and keys (CSA: index_heads x
    index_head_dim, csa.py:21-24,39-40; HCA: one head of width d_model,
    hca.py:24-25,36-37), scores q.k / sqrt(Dh) in fp32 (csa.py:58,190;
    hca.py:48,131);
  * values: one stream of width d_model shared by the heads (csa.py:25,41;
    hca.py:26,38);
  * local branch: each head's softmax over the last ``window`` tokens, the
    current one included (csa.py:55-65,185-190; hca.py:46-55,119-131), the
    heads' probabilities averaged (csa.py:74-75,203-206) and applied to the
    values;
  * memory branch: every complete block of ``ratio`` tokens is summarised by
    the compressor's key and value projections of the block mean
    (compressed_attention.py:109-123), visible from the block's last token on
    (:118-122; csa.py:94,242; hca.py:79,171).  Each head scores the visible
    summaries and takes a softmax over all of them (``top_k`` None: HCA's dense
    global attention, hca.py:84-87,175-178) or over its ``top_k`` best
    (csa.py:99-105,247-253; hca.py:88-93,179-184: k = min(top_k, entries),
    entries that are not visible weigh 0, no visible entry gives 0); heads
    averaged (csa.py:131,257) and applied to the summaries' values;
  * output: out(local_out(local) + remote_out(memory)) (csa.py:132,258;
    hca.py:101,192).

``forward`` is the sequence path from an empty state (csa.py:35-155,
hca.py:32-104).  ``step`` is the decode path (csa.py:157-259, hca.py:106-193):
the state keeps the last window - 1 keys and values with a validity flag (the
reference keeps the inputs and re-projects them, model.py:335-347, which is the
same rows), a memory that gains one entry per step (position -1 unless the step
completes a block, compressed_attention.py:192-200), and the running sum and
count of the incomplete block (:177-207).  A summary is emitted at the token
that completes a block, with that token's position.  ``reset_rows`` follows
model/recurrent_state.py:219-244 for one row.

``act_round`` rounds activations where the engine stores them in bf16 (q, k,
v, the block means, the summaries, the branch outputs and their projection);
identity gives the plain fp32 computation.  Top-k ties keep the lower index.
"""
from __future__ import annotations

import math

import torch


def _ident(t: torch.Tensor) -> torch.Tensor:
    return t


def head_scores(q: torch.Tensor, k: torch.Tensor, H: int, Dh: int) -> torch.Tensor:
    """q [B, T, H*Dh], k [B, S, H*Dh] -> scores [B, H, T, S] = q_h.k_h / sqrt(Dh),
    accumulated in fp64, returned fp32."""
    B, T = q.shape[:2]
    S = k.shape[1]
    qh = q.double().reshape(B, T, H, Dh).permute(0, 2, 1, 3)
    kh = k.double().reshape(B, S, H, Dh).permute(0, 2, 3, 1)
    return ((qh @ kh) / math.sqrt(Dh)).float()


def topk_keep(s: torch.Tensor, top_k: int) -> torch.Tensor:
    """[B, H, T, S] mask of each row's top_k entries (stable: ties keep the
    lower index), -inf entries included when fewer are finite."""
    k = min(int(top_k), s.shape[-1])
    order = torch.sort(s, dim=-1, descending=True, stable=True).indices
    keep = torch.zeros_like(s, dtype=torch.bool)
    keep.scatter_(-1, order[..., :k], True)
    return keep


def head_mean_probs(scores: torch.Tensor, visible: torch.Tensor,
                    top_k: int | None = None, keep: torch.Tensor | None = None) -> torch.Tensor:
    """scores [B, H, T, S], visible [B, T, S] -> the heads' mean of each head's
    softmax over its visible entries (``top_k`` None) or over the top_k highest
    of all S entries (invisible ones weigh 0), [B, T, S] fp32.  A row with no
    visible (selected) entry gives 0.  ``keep`` [B, H, T, S] replaces the top-k
    selection with a given one (a replayed discrete decision)."""
    s = scores.double().masked_fill(~visible[:, None], -math.inf)
    if keep is not None:
        s = s.masked_fill(~keep, -math.inf)
    elif top_k is not None:
        s = s.masked_fill(~topk_keep(s, top_k), -math.inf)
    m = s.amax(-1, keepdim=True)
    e = torch.exp(s - torch.where(torch.isfinite(m), m, torch.zeros_like(m)))
    den = e.sum(-1, keepdim=True)
    p = torch.where(den > 0, e / den.clamp_min(1e-300), torch.zeros_like(e))
    return p.mean(1).float()


def band_visible(T: int, window: int) -> torch.Tensor:
    """[T, T]: key j is in query t's window when 0 <= t - j < window."""
    t = torch.arange(T)
    d = t[:, None] - t[None, :]
    return (d >= 0) & (d < window)


def compress_sequence(h: torch.Tensor, ratio: int):
    """The compressor's sequence path for one segment (compressed_attention.py:
    105-123): means [B, n, D] of the n = T // ratio complete blocks, their
    positions (block end, [n]), and the incomplete tail's sum [B, D] and count."""
    B, T, D = h.shape
    n = T // ratio
    means = h[:, :n * ratio].reshape(B, n, ratio, D).double().mean(2).float()
    pos = torch.arange(n, dtype=torch.long) * ratio + ratio - 1
    tail = h[:, n * ratio:].double().sum(1).float()
    return means, pos, tail, T - n * ratio


class CompressedMixer:
    """One CSA or HCA mixer.  ``w`` holds fp32 weights under
    ``prefix + {cmp_wq, cmp_wk, cmp_wv, cmp_wlo, cmp_wro, cmp_wout, cmp_wck,
    cmp_wcv}`` = query, key, value, local_out, remote_out (HCA: global_out),
    out, compressor.key, compressor.value."""

    NAMES = ("cmp_wq", "cmp_wk", "cmp_wv", "cmp_wlo", "cmp_wro", "cmp_wout", "cmp_wck",
             "cmp_wcv")

    def __init__(self, w: dict, prefix: str, heads: int, head_dim: int, window: int,
                 ratio: int, top_k: int | None, act_round=None):
        self.w = {n: w[prefix + n].float() for n in self.NAMES}
        self.H, self.Dh = int(heads), int(head_dim)
        self.window, self.ratio = int(window), int(ratio)
        self.top_k = None if top_k is None else int(top_k)
        self.rnd = act_round or _ident
        # Discrete-decision forcing (verification aid, like HybridOracle's
        # forced_routes): a FIFO of [B, H, k] summary positions (-1: none), one
        # per ``step`` call; the step then uses those summaries instead of its
        # own top-k and records in sel_gaps, for each (row, head) whose choice
        # differed, its own k-th best score minus the forced set's lowest.
        self.forced_sel: list | None = None
        self.sel_gaps: list[float] = []
        self.sel_total = 0

    def _proj(self, h: torch.Tensor):
        w, rnd = self.w, self.rnd
        return rnd(h @ w["cmp_wq"].t()), rnd(h @ w["cmp_wk"].t()), rnd(h @ w["cmp_wv"].t())

    def _summaries(self, mean: torch.Tensor):
        w, rnd = self.w, self.rnd
        m = rnd(mean)
        return rnd(m @ w["cmp_wck"].t()), rnd(m @ w["cmp_wcv"].t())

    def _out(self, local: torch.Tensor, remote: torch.Tensor) -> torch.Tensor:
        w, rnd = self.w, self.rnd
        y = rnd(rnd(local) @ w["cmp_wlo"].t() + rnd(remote) @ w["cmp_wro"].t())
        return y @ w["cmp_wout"].t()

    # ---- sequence path ----------------------------------------------------
    def forward(self, h: torch.Tensor):
        """h [B, T, D] (the mixer's normalised input) from an empty state ->
        (output [B, T, D], state after the sequence, branch outputs dict)."""
        B, T, D = h.shape
        H, Dh = self.H, self.Dh
        q, k, v = self._proj(h)
        P = head_mean_probs(head_scores(q, k, H, Dh),
                            band_visible(T, self.window)[None].expand(B, T, T))
        local = (P.double() @ v.double()).float()
        means, mpos, tail, cnt = compress_sequence(h, self.ratio)
        mk, mv = self._summaries(means)
        n = mk.shape[1]
        if n:
            vis = (mpos[None, :] <= torch.arange(T)[:, None])[None].expand(B, T, n)
            Pm = head_mean_probs(head_scores(q, mk, H, Dh), vis, self.top_k)
            remote = (Pm.double() @ mv.double()).float()
        else:
            remote = torch.zeros(B, T, D)
        out = self._out(local, remote)
        Wm = self.window - 1
        st = self.new_state(B, D)
        take = min(Wm, T)
        if take:
            st["lk"][:, Wm - take:] = k[:, T - take:]
            st["lv"][:, Wm - take:] = v[:, T - take:]
            st["lvalid"][:, Wm - take:] = True
        st["mk"], st["mv"] = mk.clone(), mv.clone()
        st["mpos"] = mpos[None].expand(B, n).clone()
        st["psum"] = tail.clone()
        st["pcnt"] = torch.full((B,), cnt, dtype=torch.long)
        return out, st, {"local": local, "remote": remote, "mk": mk, "mv": mv}

    # ---- decode path ------------------------------------------------------
    def new_state(self, B: int, D: int) -> dict:
        Kw, Wm = self.H * self.Dh, self.window - 1
        return {"lk": torch.zeros(B, Wm, Kw), "lv": torch.zeros(B, Wm, D),
                "lvalid": torch.zeros(B, Wm, dtype=torch.bool),
                "mk": torch.zeros(B, 0, Kw), "mv": torch.zeros(B, 0, D),
                "mpos": torch.zeros(B, 0, dtype=torch.long),
                "psum": torch.zeros(B, D), "pcnt": torch.zeros(B, dtype=torch.long)}

    def step(self, h: torch.Tensor, st: dict, pos: torch.Tensor) -> torch.Tensor:
        """One token per row: h [B, D] at absolute positions pos [B]; updates st."""
        B, D = h.shape
        H, Dh = self.H, self.Dh
        q, k, v = self._proj(h)
        keys = torch.cat([st["lk"], k[:, None]], 1)
        vals = torch.cat([st["lv"], v[:, None]], 1)
        valid = torch.cat([st["lvalid"], torch.ones(B, 1, dtype=torch.bool)], 1)
        P = head_mean_probs(head_scores(q[:, None], keys, H, Dh), valid[:, None])
        local = (P.double() @ vals.double()).float()[:, 0]
        st["lk"], st["lv"], st["lvalid"] = keys[:, 1:], vals[:, 1:], valid[:, 1:]
        # the compressor step: the running block sum and count, a summary from
        # the mean every step, kept (visible) only when the block completes
        st["psum"] = st["psum"] + h
        st["pcnt"] = st["pcnt"] + 1
        emitted = st["pcnt"] >= self.ratio
        mean = st["psum"] / st["pcnt"].clamp_min(1).float()[:, None]
        mk, mv = self._summaries(mean)
        st["mk"] = torch.cat([st["mk"], mk[:, None]], 1)
        st["mv"] = torch.cat([st["mv"], mv[:, None]], 1)
        st["mpos"] = torch.cat([st["mpos"], torch.where(emitted, pos.long(),
                                                        torch.full_like(pos.long(), -1))[:, None]],
                               1)
        st["psum"] = torch.where(emitted[:, None], torch.zeros_like(st["psum"]), st["psum"])
        st["pcnt"] = torch.where(emitted, torch.zeros_like(st["pcnt"]), st["pcnt"])
        vis = ((st["mpos"] >= 0) & (st["mpos"] <= pos.long()[:, None]))[:, None]
        sc = head_scores(q[:, None], st["mk"], H, Dh)
        keep = None
        if self.top_k is not None and self.forced_sel:
            keep = self._forced_keep(sc, vis, st["mpos"], self.forced_sel.pop(0))
        Pm = head_mean_probs(sc, vis, self.top_k, keep=keep)
        remote = (Pm.double() @ st["mv"].double()).float()[:, 0]
        return self._out(local, remote)

    def _forced_keep(self, sc, vis, mpos, forced) -> torch.Tensor:
        """The keep mask [B, H, 1, S] of forced positions [B, H, k] (summaries
        whose position is listed), recording the gaps of differing choices."""
        forced = torch.as_tensor(forced).long()
        keep = ((mpos[:, None, :, None] == forced[:, :, None, :]) & (forced[:, :, None, :] >= 0)
                ).any(-1)[:, :, None] & vis[:, None]
        s = sc.double().masked_fill(~vis[:, None], -math.inf)
        own = topk_keep(s, self.top_k) & torch.isfinite(s)
        for b in range(s.shape[0]):
            for h in range(s.shape[1]):
                self.sel_total += 1
                only_own, only_forced = own[b, h] & ~keep[b, h], keep[b, h] & ~own[b, h]
                if not (only_own.any() or only_forced.any()):
                    continue
                if only_own.any() and only_forced.any():
                    self.sel_gaps.append(float(s[b, h][only_own].max() - s[b, h][only_forced].min()))
                else:   # the forced set is not a swap of the own one's entries
                    self.sel_gaps.append(math.inf)
        return keep

    @staticmethod
    def reset_rows(st: dict, rows: torch.Tensor) -> None:
        """Rows starting a new sequence: local history invalid, pending block
        cleared, memory entries invisible (model/recurrent_state.py:219-244)."""
        rows = rows.to(torch.bool)
        st["lvalid"] = st["lvalid"].clone()
        st["lvalid"][rows] = False
        st["psum"] = st["psum"].clone()
        st["psum"][rows] = 0
        st["pcnt"] = st["pcnt"].clone()
        st["pcnt"][rows] = 0
        st["mpos"] = st["mpos"].clone()
        st["mpos"][rows] = -1
