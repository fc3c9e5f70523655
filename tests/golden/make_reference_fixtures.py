"""Writes the golden artifact fixtures under tests/golden/ with the REFERENCE's own writers.

Run in the build container only (it imports python/zcgvs_tools from the reference checkout at
/root/reference, which does not exist where the tests run); the tests read the committed files:

    python tests/golden/make_reference_fixtures.py

What it writes (all tiny, data only):
  - ref_matrix.npy                the float32 [6, 40] matrix the embedding fixtures encode
  - ref_{float32,float16,int8,binary}.zcve
                                  formats.write_embeddings (python/zcgvs_tools/formats.py:113-149)
                                  of that matrix in each storage form
  - ref_vocab.txt, ref_docs.json  a WordPiece vocabulary and six documents
  - ref_corpus.zcvm               formats.write_metadata of the documents (formats.py:204-218)
  - ref_index.zcvl                build_lexical.main over them with its built-in WordPiece pass
                                  (build_lexical.py:105-175; BM25 k1 = 1.2, b = 0.75)
  - ref_tokens.json               the reference tokenizer's ids of every document, the
                                  input to the index's term counts
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REFERENCE_TOOLS = Path("/root/reference/python")

VOCAB = ["[PAD]", "[UNK]", "[CLS]", "[SEP]", ".", ",", "-", "the", "gpu", "search", "vector",
         "##s", "##ing", "scan", "zero", "copy", "rank", "re", "top", "k", "memory", "band",
         "##width", "fast", "int", "##8", "query", "index", "docs", "a", "of", "and", "to",
         "hbm", "cosine", "score", "bm", "##25", "lex", "##ical", "dense", "hybrid", "fuse"]

DOCS = [
    "The GPU scans vectors: zero-copy search!",
    "Re-ranking the top-k vectors, fast.",
    "HBM bandwidth and memory of a GPU; int8 queries.",
    "BM25 lexical scores fuse with dense cosine scores (hybrid search).",
    "Index of docs - search, search, search.",
    "Überfast query-ing of a zero copy index",
]


def main() -> int:
    if not REFERENCE_TOOLS.exists():
        print(f"reference tools not found at {REFERENCE_TOOLS}; fixtures left as committed")
        return 1
    sys.path.insert(0, str(REFERENCE_TOOLS))
    from zcgvs_tools import build_lexical, formats  # the reference's modules

    rng = np.random.default_rng(20261202)
    matrix = rng.standard_normal((6, 40)).astype(np.float32)
    matrix /= np.linalg.norm(matrix, axis=1, keepdims=True).astype(np.float32)
    matrix[0, :3] = [0.0, -0.0, 1e-9]  # sign-bit cases for the binary form
    np.save(HERE / "ref_matrix.npy", matrix, allow_pickle=False)
    for dtype in ("float32", "float16", "int8", "binary"):
        formats.write_embeddings(HERE / f"ref_{dtype}.zcve", matrix, normalized=True, dtype=dtype)

    (HERE / "ref_vocab.txt").write_text("".join(token + "\n" for token in VOCAB), encoding="utf-8")
    (HERE / "ref_docs.json").write_text(json.dumps(DOCS, ensure_ascii=False, indent=1), encoding="utf-8")
    formats.write_metadata(HERE / "ref_corpus.zcvm", [f"doc-{i}" for i in range(len(DOCS))], DOCS)
    encode = build_lexical.build_tokenizer(HERE / "ref_vocab.txt", None)
    tokens = [encode(text) for text in DOCS]
    (HERE / "ref_tokens.json").write_text(json.dumps(tokens), encoding="utf-8")
    argv = sys.argv
    try:
        sys.argv = ["build_lexical", "--metadata", str(HERE / "ref_corpus.zcvm"), "--vocab",
                    str(HERE / "ref_vocab.txt"), "--output", str(HERE / "ref_index.zcvl")]
        build_lexical.main()
    finally:
        sys.argv = argv
    print("fixtures written to", HERE)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
