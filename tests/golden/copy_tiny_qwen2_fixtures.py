"""Copies the reference's own tiny-model fixtures (data files its tests hold)
into tests/golden/tiny_qwen2/ and writes their sha256 manifest.

  tiny_qwen2.gguf                  tests/fixtures/tiny_qwen2.gguf (F32 weights,
                                   2 layers, n_embd 8, 2 Q / 1 KV heads,
                                   head_dim 4; made by
                                   scripts/make_tiny_qwen2_fixture.py)
  tiny_qwen2_q8_0.gguf             tests/fixtures/tiny_qwen2_q8_0.gguf (Q8_0
                                   weights, n_embd 32, 1 head, head_dim 32;
                                   tests/test_model_qwen2.cpp:241-288's model)
  stage1_golden_prefill/*.{bin,shape}
                                   the dump of a 5-token prefill of ids 0..4
  stage1_golden_decode/*.{bin,shape}
                                   the dump of the n_past 5 call for id 5 after
                                   a silent prefill of ids 0..4
                                   (both: tests/test_graph.cpp:177-239)

Run where the reference tree exists (python3 tests/golden/copy_tiny_qwen2_fixtures.py).
"""
import hashlib
import json
import os
import shutil

REF = os.environ.get("REF", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "tiny_qwen2")


def main():
    src = os.path.join(REF, "tests", "fixtures")
    os.makedirs(OUT, exist_ok=True)
    files = ["tiny_qwen2.gguf", "tiny_qwen2_q8_0.gguf"]
    for d in ("stage1_golden_prefill", "stage1_golden_decode"):
        os.makedirs(os.path.join(OUT, d), exist_ok=True)
        for f in sorted(os.listdir(os.path.join(src, d))):
            files.append(os.path.join(d, f))
    manifest = {}
    for f in files:
        shutil.copyfile(os.path.join(src, f), os.path.join(OUT, f))
        manifest[f] = hashlib.sha256(open(os.path.join(OUT, f), "rb").read()).hexdigest()
    with open(os.path.join(OUT, "manifest.json"), "w") as fh:
        json.dump({"source": "reference tests/fixtures", "sha256": manifest}, fh, indent=1, sort_keys=True)
    print(f"copied {len(files)} files to {OUT}")


if __name__ == "__main__":
    main()
