"""Writes the golden fixtures under tests/golden/ (run on the CPU; the
oracle is the checker, see oracle/oracle.c):

  smollm3_q4_seed0_greedy128.json - the SmolLM3-3B architecture with the
      seeded synthetic Q4 weights (seed 0): SHA-256 of every generated
      weight byte (in model order), the 64-token prompt, and the oracle's
      128 greedy tokens with the top-2 logit gap of each step (the decode
      workload: positions 64..191);
  smollm3_q4_seed0_ctx2048_greedy128.json - the same model after a
      1920-token prompt: 128 greedy tokens at positions 1920..2047, the
      2048-position workload (split attention past 256 positions);
  smoke_q4_seed0_x8_greedy64.json - an 8-layer model (vocab 1000, hidden
      256) whose projection scales are multiplied by 8 (recorded as
      proj_scale), so that the layers outweigh the tied embedding and the
      greedy path visits many distinct tokens (with the generator's plain
      scales a model this small repeats one token).
Each step also records the top logit, so a consumer can tell a near-tie
(gap < 1e-4 * |top logit|) from a real disagreement.

Usage: python tests/golden/make_fixtures.py [--threads N] [--only NAME]"""
import argparse
import hashlib
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import __graft_entry__ as entry  # noqa: E402


def weights_sha256(w):
    h = hashlib.sha256()
    for ws in w.layers:
        for wt in ws:
            h.update(wt.packed.tobytes())
            h.update(wt.scales.tobytes())
    h.update(w.embed.packed.tobytes())
    h.update(w.embed.scales.tobytes())
    for g in list(w.input_norm) + list(w.post_attn_norm) + [w.final_norm]:
        h.update(g.tobytes())
    h.update(w.rope_cos.tobytes())
    h.update(w.rope_sin.tobytes())
    return h.hexdigest()


def scale_projections(w, mult):
    """Multiplies every projection's Q4 group scales by mult (binary16,
    rounded to nearest even; the embedding and the norms are unchanged)."""
    import numpy as np
    for ws in w.layers:
        for wt in ws:
            wt.scales = (wt.scales.view(np.float16).astype(np.float32) * np.float32(mult)).astype(
                np.float16).view(np.uint16)
    return w


def fixture(pkg, orc, cfg, seed, prompt_tid, prompt_len, steps, threads, rope_positions, note, proj_scale=1.0):
    t0 = time.time()
    w = pkg.synthetic_model(cfg, seed=seed, rope_positions=rope_positions)
    if proj_scale != 1.0:
        scale_projections(w, proj_scale)
    prompt = pkg.synth_tokens(seed, prompt_tid, prompt_len, cfg.vocab).tolist()
    orc.set_threads(threads)
    om = orc.OracleModel(w, kv_capacity=prompt_len + steps + 8, T=threads)
    # the greedy loop of generate_raw (generate.rs:308-322) at temperature 0
    tokens, gaps, tops = [], [], []
    logits = om.prefill(prompt)
    for i in range(steps):
        t = orc.argmax(logits)
        tokens.append(t)
        gaps.append(orc.top2_gap(logits))
        tops.append(float(logits[t]))
        if i + 1 < steps:
            logits = om.forward_decode(t)
    return {
        "description": note,
        "config": {k: getattr(cfg, k) for k in ("num_layers", "vocab", "hidden", "intermediate", "num_heads",
                                                "num_kv_heads", "head_dim", "rope_half_dim", "rope_theta")},
        "rope_positions": rope_positions,
        "seed": seed,
        "proj_scale": proj_scale,
        "prompt_tid": prompt_tid,
        "weights_sha256": weights_sha256(w),
        "prompt": prompt,
        "oracle_threads": threads,
        "greedy_tokens": [int(t) for t in tokens],
        "top2_gap": [float(g) for g in gaps],
        "top_logit": tops,
        "seconds": round(time.time() - t0, 1),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--only", default="")
    args = ap.parse_args()
    pkg, orc = entry.load_package(), entry.load_oracle()
    small = entry.smoke_config(pkg)
    small.num_layers = 8
    specs = {
        "smoke_q4_seed0_x8_greedy64.json": lambda: fixture(
            pkg, orc, small, 0, 2000, 16, 64, args.threads, 128,
            "8-layer smoke model (vocab 1000, hidden 256), seed 0, projection scales x8, 16-token prompt "
            "(synth_tokens tid 2000)", proj_scale=8.0),
        "smollm3_q4_seed0_greedy128.json": lambda: fixture(
            pkg, orc, pkg.SMOLLM3_3B, 0, 2000, 64, 128, args.threads, 2048,
            "SmolLM3-3B architecture, synthetic Q4 weights seed 0, 64-token prompt (synth_tokens tid 2000), "
            "128 greedy steps: the bench's decode workload"),
        "smollm3_q4_seed0_ctx2048_greedy128.json": lambda: fixture(
            pkg, orc, pkg.SMOLLM3_3B, 0, 2002, 1920, 128, args.threads, 2048,
            "SmolLM3-3B architecture, synthetic Q4 weights seed 0, 1920-token prompt (synth_tokens tid 2002), "
            "128 greedy steps at positions 1920..2047: the bench's 2048-context workload"),
    }
    for name, make in specs.items():
        if args.only and args.only != name:
            continue
        data = make()
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(data, f, indent=1)
        print(f"{name}: {data['seconds']} s, min gap {min(data['top2_gap']):.3g}, "
              f"{len(set(data['greedy_tokens']))} distinct tokens", flush=True)


if __name__ == "__main__":
    main()
