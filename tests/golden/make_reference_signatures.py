#!/usr/bin/env python3
"""Writes reference_signatures.json: the public signatures (name, impl
owner, parameter names and types in order, return type) of the entry points
the safe wrapper crates/ramvamp-attn keeps, read from the reference tree:

  crates/core/src/kernels/attention.rs:337-400   scratch_len, AttentionScratch
  crates/core/src/kernels/attention.rs:426-859   the twelve attention functions
  crates/core/src/kv/mod.rs:163-487              KvCache's methods

and the variants (with their field names) of KvError (kv/mod.rs:39-123) and
AttentionError (kernels/attention.rs:218-311).

    python tests/golden/make_reference_signatures.py [/root/reference]

Run where the reference is present; the JSON it writes is the fixture
tests/test_rust_wrapper.py checks the wrapper against.
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from rust_sigs import enum_variants, signatures  # noqa: E402

SPANS = [("crates/core/src/kernels/attention.rs", 337, 400), ("crates/core/src/kernels/attention.rs", 426, 859),
         ("crates/core/src/kv/mod.rs", 163, 487)]


def collect(ref: str) -> dict:
    fns = []
    for path, lo, hi in SPANS:
        with open(os.path.join(ref, path)) as f:
            for s in signatures(f.read(), lo, hi):
                s["file"] = path
                fns.append(s)
    with open(os.path.join(ref, "crates/core/src/kv/mod.rs")) as f:
        kv = enum_variants(f.read(), "KvError")
    with open(os.path.join(ref, "crates/core/src/kernels/attention.rs")) as f:
        at = enum_variants(f.read(), "AttentionError")
    return {"functions": fns, "KvError": kv, "AttentionError": at}


def main(ref: str) -> None:
    d = collect(ref)
    with open(os.path.join(HERE, "reference_signatures.json"), "w") as f:
        json.dump(d, f, indent=1)
        f.write("\n")
    print(f"{len(d['functions'])} signatures, {len(d['KvError'])} + {len(d['AttentionError'])} variants")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
