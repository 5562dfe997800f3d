"""Write the c5 golden fixture (c5_7b_int4_g64.json) from the CPU oracle.

The workload is BASELINE config 5, exactly as bench.py builds it: the
Llama-2-7B-shaped decoder (dim 4096, 32 layers, 32 heads x 128, hidden
11008, vocab 32000) with random-init N(0, 0.02) weights quantized to INT4,
group 64, scale amax/7 (seed 2024), and 128 prompt ids drawn from the same
seeded generator.  The oracle (oracle/oracle.c, the C restatement of
runq.c:320-421 with the tools/quantize_int4.py dequant) forces the prompt
and then takes the argmax for 256 more positions (runq.c:681-718), 383
forward() calls in all.

Recorded (every value is the oracle's; nothing here comes from the GPU):

* ``ids``: the id chosen after each of the 383 positions (the forced prompt
  ids for positions 0..126, then the 256 greedy ids);
* ``layers``: at positions 127 (the first greedy step), 300 and 382 (the
  last), the sha256 of the residual stream's fp32 bytes after the embedding
  and after each of the 32 layers, its first 4 values, and the sha256 and
  top-5 of the logits;
* ``image``: the checkpoint's size and the sha256 of its first and last
  64 MiB, which pin the deterministic generator's bytes.

Run in the build container (about 2 minutes on 8 cores):

    make -C oracle && python tests/golden/make_c5.py
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "llama2-min-inference_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

from llama2q import host  # noqa: E402
import oracle_py as O  # noqa: E402

SEED = 2024
N_PROMPT = 128
N_GREEDY = 256
N_POS = N_PROMPT - 1 + N_GREEDY      # positions 0..382
CHECK_POS = (127, 300, 382)
EDGE = 64 << 20


def c5_checkpoint():
    cfg = host.config_7b(seq_len=4096)
    return host.synth_checkpoint(cfg, 4, 64, seed=SEED, q4_divisor=7.0)


def c5_prompt():
    return [int(v) for v in host.uniform_ints(N_PROMPT, SEED, 100, 3, 32000)]


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def image_pins(w: np.ndarray) -> dict:
    return {"bytes": int(w.nbytes), "head_sha256": sha(w[:EDGE]), "tail_sha256": sha(w[-EDGE:])}


def layer_record(xl: np.ndarray, lg: np.ndarray) -> dict:
    top = np.argsort(-lg, kind="stable")[:5]
    return {"x_sha256": [sha(row) for row in xl],
            "x_first4": [[float(v) for v in row[:4]] for row in xl],
            "logits_sha256": sha(lg),
            "top5": [[int(i), float(lg[i])] for i in top]}


def main():
    t0 = time.time()
    ck = c5_checkpoint()
    prompt = c5_prompt()
    orc = O.Oracle(ck.cfg.as_list(), ck.weights, 4, 64, max_t=N_POS)
    ids, layers = [], {}
    token = prompt[0]
    for pos in range(N_POS):
        if pos in CHECK_POS:
            xl, lg = orc.forward(token, pos, layers=True)
            layers[str(pos)] = layer_record(xl, lg)
        else:
            lg = orc.forward(token, pos)
        nxt = prompt[pos + 1] if pos < N_PROMPT - 1 else O.argmax(lg)
        ids.append(int(nxt))
        token = nxt
        if pos % 64 == 0:
            print(f"pos {pos}  {time.time() - t0:.0f}s", flush=True)
    orc.close()
    out = {"config": "Llama-2-7B shape (dim 4096, 32 layers, 32x128 heads, hidden 11008, vocab 32000), "
                     "INT4 group 64 amax/7, synth seed 2024",
           "seed": SEED, "prompt": prompt, "n_positions": N_POS, "ids": ids, "layers": layers,
           "image": image_pins(ck.weights), "generator": "oracle/oracle.c orc_forward (runq.c:320-421)"}
    with open(os.path.join(HERE, "c5_7b_int4_g64.json"), "w") as f:
        json.dump(out, f, indent=0)
    print(f"wrote c5_7b_int4_g64.json in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
