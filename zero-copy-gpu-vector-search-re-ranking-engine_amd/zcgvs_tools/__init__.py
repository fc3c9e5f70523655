"""Host-side artifact tools: the reference's file formats (ZCVE embeddings, ZCVM metadata, ZCVL
BM25 index) in NumPy, the storage encodings, and a BM25 index builder over term-id documents."""

from . import formats, lexical  # noqa: F401
