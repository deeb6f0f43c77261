"""Greedy generation on the device-resident Qwen2 engine (include/mi_hip_qwen2.h).

Mirrors the reference CLI's generation mode (src/main.cpp:209-501): load a
GGUF, prefill the prompt ids in one forward call with only the last position's
logits, then greedy-decode one token per call, printing each id on its own
line (stdout carries only ids). `--bench` times the prefill call and the
decode calls separately and prints one line of rates, as the reference's
--bench does (src/main.cpp:392-419), plus the attention kernels' share.

    python qwen2.py model.gguf --prompt-ids ids.txt [-c 2048] [-n 256] [--bench]
"""
import argparse
import ctypes
import os
import sys
import time

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import mi_hip_attn as mh  # noqa: E402


class Qwen2:
    """One loaded model with its KV cache (mi_qwen2_model + mi_kv_cache)."""

    def __init__(self, path, n_ctx=2048, max_tokens=0, device=0, lib=None):
        self.lib = lib or mh.lib()
        self.lib.init(device)
        h = ctypes.c_void_p()
        self.lib.check(self.lib.mi_hip_qwen2_load(os.fsencode(path), n_ctx, max_tokens, ctypes.byref(h)))
        self.h = h.value
        hp = mh.Qwen2Hparams()
        self.lib.check(self.lib.mi_hip_qwen2_get_hparams(self.h, ctypes.byref(hp)))
        self.hp = hp
        self.n_ctx = n_ctx
        self.n_past = 0

    def close(self):
        if self.h:
            self.lib.check(self.lib.mi_hip_qwen2_free(self.h))
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def forward(self, tokens, n_past=None, last_logits_only=True, want_logits=False):
        """One mi_qwen2_forward call; returns (next greedy id, logits or None)."""
        n_past = self.n_past if n_past is None else n_past
        ids = (ctypes.c_int32 * len(tokens))(*tokens)
        rows = 1 if last_logits_only else len(tokens)
        logits = (ctypes.c_float * (rows * self.hp.n_vocab))() if want_logits else None
        nxt = ctypes.c_int32()
        self.lib.check(self.lib.mi_hip_qwen2_forward(
            self.h, ids, len(tokens), n_past, 1 if last_logits_only else 0,
            logits if logits is not None else None, ctypes.byref(nxt)))
        return nxt.value, logits

    def set_attention(self, mode):
        """mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER (the default up to n_ctx 32768: token ids equal
        to the reference engine's) or mh.MI_HIP_QWEN2_ATTN_FUSED (the throughput kernels)."""
        self.lib.check(self.lib.mi_hip_qwen2_set_attention(self.h, mode))

    def set_timing(self, on):
        self.lib.check(self.lib.mi_hip_qwen2_set_timing(self.h, 1 if on else 0))

    def timing(self):
        a, f, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int64()
        self.lib.check(self.lib.mi_hip_qwen2_get_timing(self.h, ctypes.byref(a), ctypes.byref(f),
                                                        ctypes.byref(n)))
        return a.value, f.value, n.value

    def generate_device(self, prompt, n_predict):
        """The same loop with every step on the device (mi_hip_qwen2_generate):
        each step's embedding reads the previous greedy id from device memory,
        so no host round trip separates the steps. Same ids as generate()."""
        ids = (ctypes.c_int32 * len(prompt))(*prompt)
        out = (ctypes.c_int32 * max(1, n_predict))()
        n = ctypes.c_int32()
        self.lib.check(self.lib.mi_hip_qwen2_generate(self.h, ids, len(prompt), n_predict, out,
                                                      ctypes.byref(n)))
        self.n_past = len(prompt) + max(0, n.value - 1)
        return list(out[:n.value])

    def generate(self, prompt, n_predict, on_token=None):
        """The reference's generation loop (src/main.cpp:474-495): n_predict ids,
        the first from the prefill call, stopping early at n_ctx."""
        nxt, _ = self.forward(prompt, n_past=0)
        self.n_past = len(prompt)
        out = []
        for step in range(n_predict):
            out.append(nxt)
            if on_token:
                on_token(nxt)
            if step + 1 == n_predict or self.n_past >= self.n_ctx:
                break
            nxt, _ = self.forward([nxt], n_past=self.n_past)
            self.n_past += 1
        return out


def teacher_forced(fused, ref, prompt, ids):
    """Runs two engines in lockstep on the same history -- the prompt, then
    ids[0..i) one token per call (teacher forcing) -- and compares each step's
    last-position logits. Returns one record per step i (the logits that pick
    ids[i]): the reference engine's argmax and its top-1/top-2 margin, the
    other engine's argmax, and the largest logit difference. This is the fork
    classification of the reference's own divergence analysis
    (docs/stage1.md:118-132): a step where the argmaxes differ is a near-tie
    when its margin is within the logit differences, not a wrong history."""
    import numpy as np

    def step(tokens, n_past):
        out = []
        for m in (fused, ref):
            _, logits = m.forward(tokens, n_past=n_past, want_logits=True)
            out.append(np.frombuffer(logits, dtype=np.float32).copy())
        return out

    recs = []
    for i in range(len(ids)):
        lf, lr = step(prompt, 0) if i == 0 else step([ids[i - 1]], len(prompt) + i - 1)
        top2 = np.argpartition(lr, -2)[-2:]
        a, b = (top2[0], top2[1]) if lr[top2[0]] >= lr[top2[1]] else (top2[1], top2[0])
        recs.append(dict(step=i, ref_id=int(np.argmax(lr)), fused_id=int(np.argmax(lf)),
                         margin=float(lr[a] - lr[b]), max_diff=float(np.abs(lf - lr).max())))
    return recs


def fork_summary(recs, free_running_ids, ref_ids):
    """The numbers that classify the forks of a free-running generation
    against the reference's ids, from teacher_forced records."""
    flips = [r for r in recs if r["fused_id"] != r["ref_id"]]
    first = next((i for i, (a, b) in enumerate(zip(free_running_ids, ref_ids)) if a != b), None)
    out = dict(steps=len(recs), teacher_forced_flips=len(flips),
               flip_steps=[r["step"] for r in flips],
               largest_margin_at_flip=max((r["margin"] for r in flips), default=None),
               max_logit_diff=max(r["max_diff"] for r in recs),
               median_margin=sorted(r["margin"] for r in recs)[len(recs) // 2],
               first_free_running_divergence=first)
    if first is not None and first < len(recs):
        out["margin_at_first_divergence"] = recs[first]["margin"]
        out["max_logit_diff_at_first_divergence"] = recs[first]["max_diff"]
    return out


def read_ids(path):
    with open(path) as f:
        return [int(t) for t in f.read().split()]


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("model")
    ap.add_argument("--prompt-ids", required=True)
    ap.add_argument("-c", "--ctx", type=int, default=2048)
    ap.add_argument("-n", "--n-predict", type=int, default=128)
    ap.add_argument("--bench", action="store_true")
    ap.add_argument("--attention", choices=("fused", "reference-order"), default="reference-order",
                    help="fused: the throughput kernels; reference-order: bit-identical to the "
                         "reference engine (token ids equal)")
    a = ap.parse_args(argv)
    prompt = read_ids(a.prompt_ids)
    if not prompt:
        print("--prompt-ids file has no ids", file=sys.stderr)
        return 1
    with Qwen2(a.model, n_ctx=a.ctx, max_tokens=len(prompt)) as m:
        m.set_attention(mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER if a.attention == "reference-order"
                        else mh.MI_HIP_QWEN2_ATTN_FUSED)
        if not a.bench:
            m.generate(prompt, a.n_predict, on_token=lambda t: print(t, flush=True))
            return 0
        m.set_timing(True)
        t0 = time.perf_counter()
        nxt, _ = m.forward(prompt, n_past=0)
        t1 = time.perf_counter()
        attn_pf, _, _ = m.timing()
        m.set_timing(True)
        m.n_past = len(prompt)
        steps = 0
        t2 = time.perf_counter()
        for step in range(a.n_predict):
            if step + 1 == a.n_predict or m.n_past >= a.ctx:
                break
            nxt, _ = m.forward([nxt], n_past=m.n_past)
            m.n_past += 1
            steps += 1
        t3 = time.perf_counter()
        attn_dec, fwd_dec, _ = m.timing()
        pf_ms, dec_ms = (t1 - t0) * 1e3, (t3 - t2) * 1e3
        print(f"prefill_tokens={len(prompt)} prefill_ms={pf_ms:.3f} "
              f"prefill_tok_per_s={len(prompt) / (pf_ms / 1e3):.3f} decode_tokens={steps} "
              f"decode_ms={dec_ms:.3f} decode_tok_per_s={steps / (dec_ms / 1e3) if steps else 0:.3f} "
              f"prefill_attn_ms={attn_pf:.3f} decode_attn_ms_per_token={attn_dec / max(steps, 1):.4f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
