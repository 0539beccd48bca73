"""CPU restatement of the learned speculative drafter (test infrastructure only).

Nothing in the product imports this module; tests compare the engine's drafting kernel
(`ill_ildraft_kernel`) and its host-side request preparation with it.

* `Table`: the ILDRAFT1 file (tools/draft/ildraft.py:16-53; loader ILDraft.swift:38-84).
* `prepare`: the per-request context (ILDraft.swift:110-208; ildraft.py `Drafter.begin`
  :479-537): the prompt's first 256 ids, the top-KNB TF-IDF neighbours (cosine in float64,
  score desc then doc asc; each neighbour's TAIL + output cut to 80 tokens), the copy
  candidates (prompt ids and the first id of " word" for each space-variant word, sorted,
  first 256) and the prompt-word associations (max ln-lift, count; sorted, first 1024).
* `Drafter.evaluate`: candidates, 53 features and the scorer for the next token after
  TAIL + output (k_ildraft phases A-C, Shaders.swift:540-794; ildraft.py `features`
  :540-700, `probs` :703-716), in float32 in one fixed order:
      sc = b2; sc += WL[i] * f[i] (i = 0..52);
      per hidden unit h: a = b1[h]; a += W1[h][i] * f[i] (i = 0..52); sc += W2[h] * relu(a)
  with every product and sum rounded to float32 (no fused multiply-add), and logarithms /
  exponentials evaluated in float64 and rounded to float32.
* `Drafter.chain` / `Drafter.tree`: the drafts of one pass (k_ildraft phase D,
  Shaders.swift:795-873; ildraft.py `chain` :718-731, `tree` :733-757): the chain appends
  the best candidate (score desc, token asc) until K drafts, no candidate or a stop token;
  the tree expands best-first (cumulative probability desc, insertion order asc) with the
  top 8 children of each expanded node, the probabilities p = exp(s - m) / Z with
  m = max(best, 0) and Z = exp(-m) + the sum over the candidates, summed in float64 and
  rounded to float32 (so the order of the candidates does not matter).

Where the engine differs from the Python drafter, the engine is followed: the output window
is the last 256 committed tokens plus the drafts, neighbour sequences are cut to 80 tokens,
the context keeps the first 256 prompt ids and copy candidates and 1024 associations
(`Req(python=True)` drops these caps), at most 32 prompt-lookup occurrences and 6
continuations per n-gram order are candidates,
the edited-neighbour and association-candidate options are not used, neighbour scores enter
the features as float32. Candidates outside the model's vocabulary are dropped (a table
built for the full 151936-token vocabulary never has one).
"""
from __future__ import annotations

import math
import struct
from collections import defaultdict

import numpy as np

TAIL = (151645, 198, 151644, 77091, 198)
STOPS = (151645, 151643)
NF = 53
MAXP, MAXCOPY, MAXNB, NBSEQ, MAXAS = 256, 256, 16, 80, 1024
OB_MAX = 256
F32 = np.float32

_FNV_OFF = 0xCBF29CE484222325
_FNV_PRIME = 0x100000001B3
_M64 = (1 << 64) - 1


def fnv1a64(b: bytes) -> int:
    h = _FNV_OFF
    for x in b:
        h = ((h ^ x) * _FNV_PRIME) & _M64
    return h


def ctx_key(ctx) -> int:
    return fnv1a64(bytes([len(ctx)]) + struct.pack(f"<{len(ctx)}I", *[t & 0xFFFFFFFF for t in ctx]))


def prompt_words(text: str):
    out, seen, cur = [], set(), bytearray()
    for c in text.encode("utf-8") + b"\0":
        if 65 <= c <= 90:
            c += 32
        if 97 <= c <= 122 or 48 <= c <= 57:
            cur.append(c)
            continue
        if cur:
            w = bytes(cur)
            if w not in seen:
                seen.add(w)
                out.append(w)
            cur = bytearray()
    return out


def spacevar_words(text: str):
    ok = set(b"ABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz0123456789_.-/~:@")
    out, cur = [], bytearray()
    for c in text.encode("utf-8") + b"\0":
        if c in ok:
            cur.append(c)
            continue
        if cur:
            out.append(cur.decode("ascii"))
            cur = bytearray()
    return out


def _logf(x) -> np.float32:
    return F32(math.log(float(x)))


def _expf(x) -> np.float32:
    return F32(math.exp(float(x)))


class Table:
    def __init__(self, blob: bytes):
        h = struct.unpack_from("<8sII12I", blob, 0)
        assert h[0] == b"ILDRAFT1" and h[1] == 1, "not an ILDRAFT1 table"
        nsec = h[2]
        self.N, self.M, self.KNB, self.MAXM, self.F, self.H = h[3:9]
        self.D, self.flags = h[10], h[11]
        assert self.F == NF and self.N <= 6 and self.M <= 7 and self.KNB <= MAXNB and self.MAXM <= 12 and self.H <= 32
        sec = {}
        for i in range(nsec):
            tag, cnt, off = struct.unpack_from("<4sIQ", blob, 64 + 16 * i)
            sec[tag.decode()] = (cnt, off)
        self.sec = sec

        def arr(tag, dt):
            cnt, off = sec[tag]
            return np.frombuffer(blob, dtype=dt, count=cnt, offset=off)
        keys = arr("NGKY", "<u8")
        vl = np.frombuffer(blob, "<u4", 2 * sec["NGVL"][0], sec["NGVL"][1]).reshape(-1, 2)
        self.ng = {int(k): (int(v[0]), int(v[1])) for k, v in zip(keys, vl)}
        self.ngnx = np.frombuffer(blob, "<u4", 2 * sec["NGNX"][0], sec["NGNX"][1]).reshape(-1, 2)
        wk = arr("WDKY", "<u8")
        wv = np.frombuffer(blob, np.dtype([("idf", "<f4"), ("first", "<u4"), ("n", "<u4")]), sec["WDVL"][0], sec["WDVL"][1])
        self.words = {int(k): (F32(e["idf"]), int(e["first"]), int(e["n"])) for k, e in zip(wk, wv)}
        self.post = arr("POST", "<u4")
        self.dnrm = arr("DNRM", "<f4")
        sqof = arr("SQOF", "<u4")
        sqtk = arr("SQTK", "<u4").astype(np.int64)
        self.seqs = [[int(t) for t in sqtk[sqof[i]:sqof[i + 1]]] for i in range(len(sqof) - 1)]
        pair = np.dtype([("t", "<u4"), ("v", "<f4")])
        self.prop = {int(e["t"]): F32(e["v"]) for e in np.frombuffer(blob, pair, sec["CPTK"][0], sec["CPTK"][1])}
        self.cc1 = {int(e["t"]): F32(e["v"]) for e in np.frombuffer(blob, pair, sec["CPC1"][0], sec["CPC1"][1])}
        c2 = np.frombuffer(blob, np.dtype([("k", "<u8"), ("v", "<f4"), ("z", "<u4")]), sec["CPC2"][0], sec["CPC2"][1])
        self.cc2 = {int(e["k"]): F32(e["v"]) for e in c2}
        self.assoc = {}
        if self.flags & 1 and "ASWK" in sec:
            awk = arr("ASWK", "<u8")
            awv = np.frombuffer(blob, "<u4", 2 * sec["ASWV"][0], sec["ASWV"][1]).reshape(-1, 2)
            atk = np.frombuffer(blob, pair, sec["ASTK"][0], sec["ASTK"][1])
            self.assoc = {int(k): [(int(atk[j]["t"]), F32(atk[j]["v"])) for j in range(v[0], v[0] + v[1])]
                          for k, v in zip(awk, awv)}
        self.tflg = np.zeros(151936, np.uint8)
        tf = np.frombuffer(blob, "<u4", 2 * sec["TFLS"][0], sec["TFLS"][1]).reshape(-1, 2)
        for t, v in tf:
            if t < 151936:
                self.tflg[t] = v
        mlp = arr("MLP0", "<f4")
        H = self.H
        self.W1 = mlp[:H * NF].reshape(H, NF).astype(F32)
        self.b1 = mlp[H * NF:H * NF + H].astype(F32)
        self.W2 = mlp[H * NF + H:H * NF + 2 * H].astype(F32)
        self.b2 = F32(mlp[H * NF + 2 * H])
        self.WL = mlp[H * NF + 2 * H + 1:H * NF + 2 * H + 1 + NF].astype(F32)

    @staticmethod
    def load(path):
        with open(path, "rb") as f:
            return Table(f.read())


class Req:
    """The per-request context (ILDraft.swift:110-208)."""

    def __init__(self, table: Table, pids, text: str, encode=None, python: bool = False):
        """python: the Python drafter's context, without the engine's caps (DraftReq,
        ILDraft.swift:20-35): all prompt ids (not the first 256), each neighbour's whole
        TAIL + output (not its first 80 tokens), every copy candidate and association (not
        the first 256 / 1024)."""
        t = table
        self.P = [int(x) for x in (pids if python else pids[:MAXP])]
        pset = set(self.P)
        words = prompt_words(text)
        score = defaultdict(float)
        q2 = 0.0
        for w in words:
            e = t.words.get(fnv1a64(w))
            if e is None:
                continue
            idf, first, n = e
            w2 = float(idf) * float(idf)
            q2 += w2
            for j in range(n):
                score[int(t.post[first + j])] += w2
        qn = math.sqrt(q2) if q2 > 0 else 1.0
        ranked = sorted(((s / (qn * float(t.dnrm[d])), d) for d, s in score.items()), key=lambda x: (-x[0], x[1]))
        self.nb = []                                  # (score f32, doc, sequence <= 80)
        for s, d in ranked[:min(t.KNB, MAXNB)]:
            seq = list(TAIL) + t.seqs[d]
            self.nb.append((F32(s), d, seq if python else seq[:NBSEQ]))
        sv = set()
        if encode is not None:
            for w in spacevar_words(text):
                ids = encode(" " + w)
                if ids and ids[0] not in pset:
                    sv.add(int(ids[0]))
        self.copy = sorted(pset | sv)
        if not python:
            self.copy = self.copy[:MAXCOPY]
        self.copy_inp = [c in pset for c in self.copy]
        amap = {}
        if t.flags & 1:
            for w in words:
                for tok, ll in t.assoc.get(fnv1a64(w), ()):
                    e = amap.get(tok)
                    amap[tok] = (max(e[0], ll), e[1] + 1) if e else (ll, 1)
        self.as_tok = sorted(amap) if python else sorted(amap)[:MAXAS]
        self.as_max = [amap[x][0] for x in self.as_tok]
        self.as_cnt = [amap[x][1] for x in self.as_tok]
        # request-constant lookups of the copy features
        self.pprop = [t.prop.get(x, F32(0.2)) for x in self.P]
        self.copy_pt = [t.prop.get(x, F32(0.2)) if inp else F32(0.3) for x, inp in zip(self.copy, self.copy_inp)]


class Drafter:
    """`py_compat`: compare the copy rate of the first-unused prompt token with 0.3 in float64
    as the Python drafter does (ildraft.py:643) instead of with 0.3f as the engine does
    (Shaders.swift:646): the two differ for a rate that rounds to float32(0.3), such as
    (1 + 0.5) / (3 + 2)."""

    def __init__(self, table: Table, req: Req, vocab: int = 151936, py_compat: bool = False):
        self.t, self.r, self.vocab, self.py_compat = table, req, vocab, py_compat

    def evaluate(self, ob, Lfull, ticks, first_out):
        """Candidates (ascending tokens) and float32 scores for the token after TAIL + ob,
        where ob = the output window (committed tokens, then drafts), Lfull = the full output
        length, ticks = the '`' count of the whole output."""
        toks, Fm = self.features(ob, Lfull, ticks, first_out)
        return toks, self.score(Fm)

    def score(self, Fm):
        """The scorer, float32 in the fixed order."""
        t = self.t
        sc = np.full(Fm.shape[0], t.b2, F32)
        for i in range(NF):
            sc = sc + t.WL[i] * Fm[:, i]
        for h in range(t.H):
            a = np.full(Fm.shape[0], t.b1[h], F32)
            for i in range(NF):
                a = a + t.W1[h, i] * Fm[:, i]
            sc = sc + t.W2[h] * np.maximum(a, F32(0))
        return sc.astype(F32)

    def features(self, ob, Lfull, ticks, first_out):
        """Candidates (ascending tokens) and their float32 feature rows."""
        t, r = self.t, self.r
        Lo = len(ob)
        L = 5 + Lo
        ctx = lambda i: TAIL[i] if i < 5 else ob[i - 5]   # noqa: E731
        # n-gram distributions, orders 1..6
        dist = {}
        for n in range(1, 7):
            if n <= t.N and n <= L:
                e = t.ng.get(ctx_key([ctx(i) for i in range(L - n, L)]))
                if e is not None:
                    tot, fn = e
                    first, cnt = fn >> 3, fn & 7
                    dist[n] = (tot, [(int(t.ngnx[first + k][0]), int(t.ngnx[first + k][1])) for k in range(cnt)])
        ln = max(dist) if dist else 0
        s3 = max([n for n, e in dist.items() if e[0] >= 3], default=0)
        s10 = max([n for n, e in dist.items() if e[0] >= 10], default=0)
        toplong, entlow = -1, False
        if ln:
            tot, top = dist[ln]
            toplong = top[0][0]
            ent = F32(0)
            for _, c in top:
                pr = F32(c) / F32(tot)
                ent = F32(ent - F32(pr * _logf(pr)))
            entlow = bool(ent < F32(0.3))
        # self-repetition: longest suffix (<= MAXM) seen earlier, latest occurrence
        self_n, self_tok = 0, -1
        best = (0, -1)
        for e in range(1, Lo):
            m, lim = 0, min(t.MAXM, Lo - 1, e)
            while m < lim and ob[e - 1 - m] == ob[Lo - 1 - m]:
                m += 1
            if m > 0 and (m, e) > best:
                best = (m, e)
        if best[0] > 0:
            self_n, self_tok = best[0], ob[best[1]]
        # prompt lookup: every occurrence (ascending, <= 32) of the longest suffix in P
        P = r.P
        pm = {}
        for e in range(1, len(P)):
            m, lim = 0, min(t.MAXM, Lo, e)
            while m < lim and P[e - 1 - m] == ob[Lo - 1 - m]:
                m += 1
            pm[e] = m
        pr_n = max(pm.values(), default=0)
        pr_e = [e for e in sorted(pm) if pm[e] == pr_n][:32] if pr_n > 0 else []
        # neighbours: longest suffix of ctx in the sequence, first occurrence
        votes = []
        for (sk, _, seq) in r.nb:
            bm, be = 0, None
            for e in range(1, len(seq)):
                m, lim = 0, min(t.MAXM, L, e)
                while m < lim and seq[e - 1 - m] == ctx(L - 1 - m):
                    m += 1
                if m > bm:
                    bm, be = m, e
            votes.append((seq[be], bm) if bm > 0 else (-1, 0))
        # copy context
        c_1, c_2 = ctx(L - 1), ctx(L - 2)
        sc1 = t.cc1.get(c_1, F32(0.1))
        sc2 = t.cc2.get(((c_2 & 0xFFFFFFFF) << 32) | (c_1 & 0xFFFFFFFF), F32(0.1))
        used = set(ob)
        firstun = -1
        for x, pp in zip(P, r.pprop):
            if x not in used and (float(pp) > 0.3 if self.py_compat else pp > F32(0.3)):
                firstun = x
                break
        # candidates
        raw = []
        for n in range(1, 7):
            if n in dist:
                raw += [tk for tk, _ in dist[n][1][:6]]
        raw.append(self_tok if self_n > 0 else -1)
        raw += [v[0] for v in votes]
        raw += [P[e] for e in pr_e]
        raw += r.copy
        toks = sorted({x for x in raw if 0 <= x < self.vocab})
        if not toks:
            return [], np.zeros((0, NF), F32)
        nnb = max(1, len(r.nb))
        Fm = np.zeros((len(toks), NF), F32)
        for ci, tok in enumerate(toks):
            f = Fm[ci]
            f[0] = 1
            for n, (tot, top) in dist.items():
                c, rank = 0, -1
                for k, (tk, cc) in enumerate(top):
                    if tk == tok:
                        c, rank = cc, k
                        break
                if n == ln and rank == 1:
                    f[13] = 1
                if n == ln and rank >= 2:
                    f[14] = 1
                if c > 0:
                    p = F32(c) / F32(tot)
                    f[6 + n] = p
                    if n == ln:
                        f[1] = p
                        f[3] = F32(F32(n) / F32(6)) * p
                        f[4] = _logf(F32(1) + F32(c))
                    if n == s3:
                        f[5] = p
                    if n == s10:
                        f[6] = p
            if tok == toplong:
                f[2] = 1
                if entlow:
                    f[15] = 1
            if self_n > 0 and tok == self_tok:
                f[16] = F32(self_n) / F32(4)
                f[17] = 1
                f[18] = 1 if self_n >= 3 else 0
            for q, e in enumerate(pr_e):
                if P[e] == tok:
                    f[19] = F32(pr_n) / F32(4)
                    f[20] = 1
                    f[21] = 1 if pr_n >= 2 else 0
                    if q == 0:
                        f[22] = 1
            nbs = nbm = nbx = F32(0)
            nbc = 0
            for k, ((sk, _, _), (vt, vn)) in enumerate(zip(r.nb, votes)):
                if vt != tok:
                    continue
                mk = F32(min(vn, 8)) / F32(8)
                nbs = F32(nbs + sk)
                nbm = F32(nbm + F32(sk * mk))
                nbc += 1
                nbx = max(nbx, mk)
                if k == 0:
                    f[27] = 1
                    f[28] = mk
            f[23], f[24], f[25], f[26] = nbs, nbm, F32(nbc) / F32(nnb), nbx
            usedt = tok in used
            inp = False
            if tok in r.copy:
                i = r.copy.index(tok)
                inp = r.copy_inp[i]
                pt = r.copy_pt[i]
                f[33] = _logf(pt / F32(F32(1) - pt)) / F32(4)
                f[34], f[35] = sc1, sc2
                f[36] = 0 if usedt else 1
                f[37] = 1 if tok == firstun else 0
                f[38] = 0 if inp else 1
            f[29] = 1 if tok in STOPS else 0
            f[30] = 1 if inp else 0
            f[31] = f[2] * min(F32(1), F32(2) * f[25])
            f[32] = f[17] * min(F32(1), F32(2) * f[25])
            f[39] = 1 if Lfull > 0 and first_out in (73594, 13874) else 0
            f[40] = 1 if Lfull > 0 and first_out == 63 else 0
            tf = int(t.tflg[tok]) if tok < 151936 else 0
            f[41] = 1 if tf & 7 else 0
            f[42] = 1 if tf & 8 else 0
            f[43] = ticks & 1
            f[44] = F32(min(Lfull, 32)) / F32(32)
            f[45] = 1 if usedt else 0
            if tok in r.as_tok:
                i = r.as_tok.index(tok)
                f[46] = r.as_max[i] / F32(4)
                f[47] = F32(min(r.as_cnt[i], 4)) / F32(4)
        return toks, Fm

    @staticmethod
    def _best(toks, sc):
        b = 0
        for i in range(1, len(toks)):
            if sc[i] > sc[b]:
                b = i
        return b

    def _state(self, out):
        have = len(out)
        ob = list(out[max(0, have - OB_MAX):])
        ticks = int(sum(int(self.t.tflg[x]) & 7 for x in out if 0 <= x < 151936))
        return ob, have, ticks

    def chain(self, out, K, eos=STOPS):
        """Up to K drafts after the committed output `out`."""
        ob, have, ticks = self._state(out)
        d = []
        while len(d) < K:
            toks, sc = self.evaluate(ob, have + len(d), ticks, out[0])
            if not toks:
                break
            bt = toks[self._best(toks, sc)]
            d.append(bt)
            ob.append(bt)
            ticks += int(self.t.tflg[bt]) & 7
            if bt in eos:
                break
        return d

    def _probs(self, toks, sc):
        b = self._best(toks, sc)
        mx = max(sc[b], F32(0))
        ez = [_expf(F32(s - mx)) for s in sc]
        Z = F32(math.fsum([float(_expf(-mx))] + [float(e) for e in ez]))
        order = sorted(range(len(toks)), key=lambda i: (-float(sc[i]), toks[i]))
        return [(toks[i], ez[i]) for i in order[:8]], Z

    def probs(self, out):
        """[(token, p)] of the next token, best first (for comparison with the reference)."""
        ob, have, ticks = self._state(out)
        toks, sc = self.evaluate(ob, have, ticks, out[0])
        if not toks:
            return []
        b = self._best(toks, sc)
        mx = max(sc[b], F32(0))
        ez = [_expf(F32(s - mx)) for s in sc]
        Z = F32(math.fsum([float(_expf(-mx))] + [float(e) for e in ez]))
        order = sorted(range(len(toks)), key=lambda i: (-float(sc[i]), toks[i]))
        return [(toks[i], float(ez[i] / Z)) for i in order]

    def tree(self, out, B, eos=STOPS):
        """Best-first tree of up to B drafts: (parents, tokens) with parent -1 = the root (the
        last committed token) and node i's parent < i."""
        ob0, have, ticks0 = self._state(out)
        base = len(ob0)
        par, tok, dep, cum = [-1], [out[-1]], [0], [F32(1)]     # row 0 = the root
        heap = []                                                # [cum, order, parent row, token]
        order = 0
        erow, depth, ob, ticks = 0, 0, list(ob0), ticks0
        for _ in range(64):
            toks, sc = self.evaluate(ob[:base + depth], have + depth, ticks, out[0])
            if toks:
                top, Z = self._probs(toks, sc)
                for tk, e in top:
                    if len(heap) < 128:
                        heap.append([F32(F32(cum[erow] * e) / Z), order, erow, tk])
                        order += 1
            go = False
            while len(par) < B + 1 and heap:
                bi = 0
                for q in range(1, len(heap)):
                    if heap[q][0] > heap[bi][0] or (heap[q][0] == heap[bi][0] and heap[q][1] < heap[bi][1]):
                        bi = q
                c, _, p, tk = heap.pop(bi)
                i = len(par)
                par.append(p)
                tok.append(tk)
                dep.append(dep[p] + 1)
                cum.append(c)
                if tk in eos or len(par) == B + 1:
                    continue
                path, rr = [], i
                while rr > 0:
                    path.append(tok[rr])
                    rr = par[rr]
                path.reverse()
                ob = ob0[:base] + path
                depth = dep[i]
                ticks = ticks0 + sum(int(self.t.tflg[x]) & 7 for x in path)
                erow = i
                go = True
                break
            if not go:
                break
        return [p - 1 for p in par[1:]], tok[1:]


def tree_rows(parents, tokens, root):
    """The pass rows of a tree (row 0 = the root): tokens, depths, parents (row indices)."""
    toks, dep, par = [root], [0], [0]
    for p, t in zip(parents, tokens):
        pr = p + 1
        toks.append(t)
        par.append(pr)
        dep.append(dep[pr] + 1)
    return toks, dep, par


def simulate(prompt, greedy, max_new, draft_fn, eos=STOPS):
    """Speculative decoding with a drafter, given the model's greedy continuation: (tokens,
    passes, accepted). draft_fn(out) -> ("chain", drafts) or ("tree", parents, tokens)."""
    out, passes, accepted = [], 0, 0
    plan = None
    while True:
        c = len(out)
        m = 0
        if plan is not None and plan[0] == "chain":
            d = plan[1]
            while m < len(d) and d[m] == greedy[c + m]:
                m += 1
        elif plan is not None:
            _, parents, tokens = plan
            cur = -1
            while True:
                nxt = -1
                for i, (p, t) in enumerate(zip(parents, tokens)):
                    if p == cur and t == greedy[c + m]:
                        nxt = i
                        break
                if nxt < 0:
                    break
                cur = nxt
                m += 1
        passes += 1
        accepted += m
        stop = False
        for k in range(m + 1):
            tok = greedy[c + k]
            out.append(tok)
            if tok in eos or len(out) >= max_new:
                stop = True
                break
        if stop:
            return out, passes, accepted
        plan = draft_fn(out)
