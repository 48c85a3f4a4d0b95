"""Writes corpus-subset.jsonl: the rows of the reference's tokenizer corpus (goldens/tokenizer/g1/cases.jsonl) that can
be checked without the Qwen3 tokenizer.json (absent here): every decode case, every encode case whose ids hold an added
token, every encode_bytes case and every encode_reject case, unchanged.

    python tests/golden/tokenizer/make_corpus_subset.py [/root/reference]
"""
import json
import os
import sys

ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
src = os.path.join(ref, "goldens", "tokenizer", "g1", "cases.jsonl")
keep = []
for line in open(src, encoding="utf-8"):
    row = json.loads(line)
    added = row["kind"] == "encode" and any(i >= 151643 for i in row["ids"])
    if row["kind"] in ("decode", "encode_bytes", "encode_reject") or added:
        keep.append(line if line.endswith("\n") else line + "\n")
with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "corpus-subset.jsonl"), "w", encoding="utf-8") as f:
    f.writelines(keep)
print(len(keep), "rows")
