"""Write golden vectors of the learned drafter from the reference's own Python drafter.

The reference's drafter specification is `tools/draft/ildraft.py` (its Swift/Metal port is
ILDraft.swift + k_ildraft). Its golden vectors (`export_swift_test.py`) need the training
outputs and the real tokenizer, which are not in the tree, so the vectors are made here:

* a synthetic corpus (tests/golden/ildraft_corpus.py) is turned into an ILDRAFT1 table by
  this package's writer (`instantllm_amd.ildraft.build`; deterministic, so the tests
  rebuild it and check its SHA-256, recorded with the vectors);
* the reference's `Tables.load` reads that file and its `Drafter` (with the corpus's
  stand-in tokenizer for the space variants) drafts for held-in and held-out requests:
  the neighbour ranking, copy candidates and associations of `begin`, and at every output
  position the top-3 probabilities of `probs` and the 7-draft `chain`, at two positions
  per request the candidates and feature rows of `features`; 15-node `tree`s at a few
  positions -> `ildraft_small.json`;
* the same recordings on the reference's own shipped table (`tools/draft/ildraft-q4.bin`:
  its real n-gram statistics, TF-IDF index, associations, token flags and trained scorer)
  for requests taken from its drafting corpus (`corpus-q4.jsonl`) -> `ildraft_real.json`
  (the table itself stays in the reference; its SHA-256 is recorded).

Only inputs and outputs are stored, never reference code; the reference is not needed at
test time. Usage: python tests/golden/make_ildraft_fixtures.py [/root/reference]
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path
from types import SimpleNamespace

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE))
from instantllm_amd import ildraft as W  # noqa: E402
from ildraft_corpus import Corpus, mock_encode  # noqa: E402

VECTORS = HERE / "ildraft_small.json"
SCORER_EMPHASIS = {1: 3.0, 2: 1.5, 17: 2.0, 20: 1.0, 23: 1.5, 36: 0.5, 29: -1.0}


def make_table():
    """(table bytes, requests to draft for): 8 of the table's own requests, 8 new ones."""
    c = Corpus(seed=0)
    recs = c.records(300)
    spec = W.TableSpec(pair_min_count=2)
    blob = W.build(recs, spec, W.random_scorer(spec.hidden, seed=5, emphasis=SCORER_EMPHASIS), c.flags)
    return blob, recs[:8] + [c.request(f) for f in range(8)]


class _Tok:
    def encode(self, text, add_special_tokens=False):
        return SimpleNamespace(ids=mock_encode(text))

    def decode(self, ids):
        raise AssertionError("token flags come from the table")


REAL_VECTORS = HERE / "ildraft_real.json"
REAL_TABLE = "tools/draft/ildraft-q4.bin"
REAL_CORPUS = "tools/draft/corpus-q4.jsonl"


def real_requests(ref_root, n=12):
    """Requests drawn from the reference's drafting corpus (real greedy outputs of its q4
    model: the table's training outputs): prompt text and output ids as recorded; the prompt
    ids are a stand-in (the tokenizer is not in the tree): the output's first distinct ids
    and the stand-in ids of the prompt's words, so that prompt-lookup and copy features fire."""
    import json as J
    from ildraft_corpus import tok_id
    lines = Path(ref_root, REAL_CORPUS).read_text().splitlines()
    out = []
    for k in range(n):
        r = J.loads(lines[(k * 1877) % len(lines)])
        y = list(r["ids"]) + ([r["stop"]] if r.get("stop", -1) in (151645, 151643) else [])
        seen = []
        for t in y:
            if t not in seen and len(seen) < 6:
                seen.append(t)
        pids = [tok_id(w) for w in r["prompt"].split()][:20] + seen
        out.append({"prompt": r["prompt"], "pids": pids, "y": y[:96]})
    return out


def real_main(ref_root, R):
    """Vectors of the reference drafter on the reference's own shipped table."""
    tab = R.Tables.load(str(Path(ref_root, REAL_TABLE)))
    d = R.Drafter(tab, _Tok())
    out = []
    for r in real_requests(ref_root):
        d.begin(r["pids"], r["prompt"])
        y = r["y"]
        pos = []
        for i in range(1, len(y)):
            pr = d.probs(y[:i])
            e = {"top": [[int(t), float(p)] for t, p in pr[:3]], "chain": [int(t) for t in d.chain(y[:i], 7)]}
            if i in (1, len(y) // 2):
                toks, rows = d.features(y[:i])
                e["feat"] = {"toks": [int(t) for t in toks], "rows": [[round(float(x), 9) for x in row] for row in rows]}
            pos.append(e)
        par, toks = d.tree(y[:2], 15)
        out.append({"prompt": r["prompt"], "pids": r["pids"], "y": y,
                    "nb_seqs": [[int(t) for t in seq] for _, seq, _ in d.nb],
                    "nb_scores": [float(s) for s, _, _ in d.nb],
                    "copy": [int(x) for x in d.copy_cands],
                    "assoc": {str(k): [float(v[0]), int(v[1])] for k, v in sorted(d.as_map.items())},
                    "pos": pos, "trees": [{"at": 2, "parents": par, "tokens": [int(t) for t in toks]}]})
    import hashlib as HL
    sha = HL.sha256(Path(ref_root, REAL_TABLE).read_bytes()).hexdigest()
    REAL_VECTORS.write_text(json.dumps({"table_sha256": sha, "requests": out}))
    print(f"real table: {len(out)} requests / {sum(len(x['pos']) for x in out)} positions -> {REAL_VECTORS.name}")


def main(ref_root="/root/reference"):
    blob, reqs = make_table()
    sys.path.insert(0, str(Path(ref_root) / "tools" / "draft"))
    import ildraft as R  # the reference drafter (read-only)
    tmp = Path("/tmp/ildraft_small.bin")
    tmp.write_bytes(blob)
    tab = R.Tables.load(str(tmp))
    d = R.Drafter(tab, _Tok())
    out = []
    for r in reqs:
        d.begin(r["pids"], r["prompt"])
        y = r["y"]
        pos = []
        for i in range(1, len(y)):
            pr = d.probs(y[:i])
            e = {"top": [[int(t), float(p)] for t, p in pr[:3]], "chain": [int(t) for t in d.chain(y[:i], 7)]}
            if i in (1, len(y) // 2):
                toks, rows = d.features(y[:i])
                e["feat"] = {"toks": [int(t) for t in toks], "rows": [[round(float(x), 9) for x in row] for row in rows]}
            pos.append(e)
        trees = []
        for i in sorted({1, max(1, len(y) // 2)}):
            par, toks = d.tree(y[:i], 15)
            trees.append({"at": i, "parents": par, "tokens": [int(t) for t in toks]})
        out.append({"prompt": r["prompt"], "pids": r["pids"], "y": y,
                    "nb_seqs": [[int(t) for t in seq] for _, seq, _ in d.nb],
                    "nb_scores": [float(s) for s, _, _ in d.nb],
                    "copy": [int(x) for x in d.copy_cands],
                    "assoc": {str(k): [float(v[0]), int(v[1])] for k, v in sorted(d.as_map.items())},
                    "pos": pos, "trees": trees})
    VECTORS.write_text(json.dumps({"table_sha256": hashlib.sha256(blob).hexdigest(), "requests": out}))
    n = sum(len(x["pos"]) for x in out)
    print(f"table {len(blob)} B; {len(out)} requests / {n} positions -> {VECTORS.name}")
    real_main(ref_root, R)


if __name__ == "__main__":
    main(*sys.argv[1:])
