"""Writes the end-to-end fixtures: greedy generation by the reference engine.

The reference's own CLI (oracle/_ref/mini_infer: src/main.cpp and the core
sources, compiled in place by oracle/Makefile) runs on the random-initialised
Qwen2.5-0.5B-shaped Q8_0 model that mini-infer-llama.cpp_amd/qwen2_gguf.py
writes from a seed:

  * 128 seeded prompt ids, prefill in one call, 256 greedy ids with n_ctx 2048
    (`mini_infer model --prompt-ids ids -c 2048 -n 256`);
  * `--dump DIR` over the same prompt: the last position's logits row (the
    prefill call's lm_head output, src/model_qwen2.cpp:645-673).

Outputs (committed): e2e_qwen05_q8_0.json (seed, model sha256, prompt, ids)
and e2e_qwen05_q8_0_logits.npz (the logits row). The model file itself
(527 MB) is not kept: tests regenerate it from the seed and check its sha256.

    python tests/golden/make_e2e_golden.py [--workdir /tmp/e2e]
"""
import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "mini-infer-llama.cpp_amd"))
import qwen2_gguf  # noqa: E402

SEED = 1234
N_PROMPT = 128
N_PREDICT = 256
N_CTX = 2048
NAME = "e2e_qwen05_q8_0"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workdir", default="/tmp/e2e")
    ap.add_argument("--threads", type=int, default=8)
    a = ap.parse_args()
    os.makedirs(a.workdir, exist_ok=True)
    subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "ref"], check=True)
    exe = os.path.join(ROOT, "oracle", "_ref", "mini_infer")
    model = os.path.join(a.workdir, "qwen05_q8_0.gguf")
    t = time.time()
    sha = qwen2_gguf.write_qwen2_q8_0(model, SEED)
    print(f"model {sha} ({time.time() - t:.1f} s)", flush=True)
    prompt = qwen2_gguf.prompt_ids(SEED, N_PROMPT, qwen2_gguf.QWEN2_05B["n_vocab"])
    ids_path = os.path.join(a.workdir, "prompt_ids.txt")
    with open(ids_path, "w") as f:
        f.write(" ".join(map(str, prompt)) + "\n")
    t = time.time()
    r = subprocess.run([exe, model, "--prompt-ids", ids_path, "-c", str(N_CTX), "-n", str(N_PREDICT),
                        "-t", str(a.threads)], check=True, capture_output=True, text=True)
    gen_s = time.time() - t
    ids = [int(x) for x in r.stdout.split()]
    assert len(ids) == N_PREDICT, len(ids)
    dump = os.path.join(a.workdir, "dump")
    os.makedirs(dump, exist_ok=True)
    subprocess.run([exe, model, "--prompt-ids", ids_path, "-c", str(N_CTX), "--dump", dump],
                   check=True, capture_output=True)
    rows, cols = map(int, open(os.path.join(dump, "logits.shape")).read().split())
    logits = np.fromfile(os.path.join(dump, "logits.bin"), dtype=np.float32).reshape(rows, cols)
    last = logits[-1].copy()
    assert int(np.argmax(last)) == ids[0]
    np.savez_compressed(os.path.join(HERE, NAME + "_logits.npz"), logits_last=last)
    top = np.sort(last)[::-1]
    meta = {
        "what": "greedy ids of the reference engine (oracle/_ref/mini_infer) on the random-init "
                "Qwen2.5-0.5B-shaped Q8_0 model of qwen2_gguf.write_qwen2_q8_0(seed)",
        "seed": SEED, "model_sha256": sha, "n_ctx": N_CTX, "n_predict": N_PREDICT,
        "prompt": prompt, "ids": ids,
        "reference_cmd": f"mini_infer MODEL --prompt-ids IDS -c {N_CTX} -n {N_PREDICT} -t {a.threads}",
        "reference_seconds": round(gen_s, 2),
        "prefill_top2_margin": float(top[0] - top[1]),
    }
    with open(os.path.join(HERE, NAME + ".json"), "w") as f:
        json.dump(meta, f, indent=1)
    print(f"ids {ids[:8]}... reference {gen_s:.1f} s, prefill top-2 margin {meta['prefill_top2_margin']:.3e}")


if __name__ == "__main__":
    main()
