"""Write golden greedy token streams of the CPU oracle for the benchmark configs.

    python tests/golden/make_golden.py tinyllama-1.1b [--decode N] [--prompt N]

Output: tests/golden/<config>_p<prompt>_d<decode>.json with the prompt ids, the greedy
stream, the per-step top-1/top-2 logit margin and a digest of the generated weights (so a
generator change is detected).  The oracle is the C++ restatement of Camelid's CPU
forward (oracle/camelid_oracle.cpp); the weights come from camelid_amd.model's seeded
generator, identical on every machine with the same glibc.
"""
import argparse
import hashlib
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from camelid_amd.model import CONFIGS, SyntheticModel, prompt_tokens  # noqa: E402
from oracle.oracle import OracleModel  # noqa: E402


def weights_digest(model) -> str:
    h = hashlib.sha256()
    for layer in model.layers:
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            h.update(layer["projs"][name][:4096].tobytes())
    h.update(model.token_embd[:4096].tobytes())
    h.update(model.output[-4096:].tobytes())
    return h.hexdigest()


def golden_path(name: str, prompt: int, decode: int) -> Path:
    return Path(__file__).resolve().parent / f"{name}_p{prompt}_d{decode}.json"


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("config", choices=sorted(CONFIGS))
    ap.add_argument("--prompt", type=int, default=None)
    ap.add_argument("--decode", type=int, default=None)
    a = ap.parse_args()
    cfg = CONFIGS[a.config]
    P = a.prompt or cfg.prompt_len
    D = a.decode or cfg.decode_len
    t0 = time.time()
    model = SyntheticModel.generate(cfg)
    prompt = prompt_tokens(cfg, P)
    orc = OracleModel(model, P + D)
    margins: list = []
    t1 = time.time()
    toks = orc.generate(prompt, D, margins)
    t2 = time.time()
    out = {
        "config": cfg.name,
        "prompt_len": P,
        "decode_len": D,
        "prompt": [int(t) for t in prompt],
        "tokens": toks,
        "margins": margins,
        "weights_sha256_prefix": weights_digest(model),
        "oracle_seconds": round(t2 - t1, 1),
        "note": "greedy stream of oracle/camelid_oracle.cpp (C++ restatement of Camelid's CPU forward)",
    }
    path = golden_path(cfg.name, P, D)
    path.write_text(json.dumps(out, indent=1))
    print(f"wrote {path} (gen {t1 - t0:.1f}s, oracle {t2 - t1:.1f}s, min margin {min(margins):.4g})")


if __name__ == "__main__":
    main()
