"""Golden fixtures for the parity tests: inputs and oracle outputs.

`python -m tests.golden.make_golden` regenerates tests/golden/*.npz from the
seeded inputs below with the CPU oracle (oracle/nsr_oracle.c). The fixtures
are small (< 1 MB in total) and committed; the GPU tests check the HIP path
against them and tests/test_oracle.py checks that the oracle still
reproduces them bit for bit.

The reference holds no fixtures or golden vectors for these ops (its GPU
self-tests in src/kokoro/gpu_decoder.rs print an error with no expected
data), so the Kokoro case uses that self-test's known-answer input
generator (gpu_decoder.rs:84-87) and the other cases seeded synthetic inputs.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

from nspeech_amd import configs
from oracle import restated as R

HERE = Path(__file__).resolve().parent


def _inputs() -> dict[str, dict[str, np.ndarray]]:
    g = configs.rng(4242)
    cases: dict[str, dict[str, np.ndarray]] = {}
    # Q8_0: small vocab, ids with repeats and both ends; d = 64 and 416
    for vocab, d, n in ((37, 64, 50), (64, 416, 40)):
        ids = g.integers(0, vocab, size=n).astype(np.uint32)
        ids[:3] = [0, vocab - 1, vocab - 1]
        cases[f"q8_v{vocab}_d{d}"] = {"blocks": configs.make_q8_0_table(g, vocab, d), "ids": ids,
                                      "vocab": np.int64(vocab), "d": np.int64(d)}
    c = configs.c0()
    cases["ln_c0_rows16"] = {"x": c["x"][0, :16].copy(), "gamma": c["gamma"], "beta": c["beta"]}
    cases["ln_unit_offset_8x288"] = {"x": (g.standard_normal((8, 288)) * 2 + 1).astype(np.float32),
                                     "gamma": (0.1 * g.standard_normal(288)).astype(np.float32)}
    cases["rope_b1h2t16_pos5"] = {"q": g.standard_normal((1, 2, 16, 64)).astype(np.float32),
                                  "rot": np.int64(32), "theta": np.float32(10000.0), "pos0": np.int64(5)}
    k = configs.kokoro_kat(4, 100)
    cases["adain_kokoro_kat_c4_t100"] = {"x": k["x"], "gamma": k["gamma"], "beta": k["beta"], "alpha": k["alpha"]}
    c = configs.c2(C=4, T=1000)
    cases["adain_c4_t1000"] = {"x": c["x"], "gamma": c["gamma"], "beta": c["beta"], "alpha": c["alpha"]}
    c = configs.c4a(rows=8)
    cases["resln_bf16_8x1024"] = {"x": c["x"], "res": c["res"], "gamma": c["gamma"], "beta": c["beta"]}
    cases["act_f32_1000"] = {"x": (g.standard_normal(1000) * 4).astype(np.float32)}
    return cases


def compute(name: str, case: dict) -> dict[str, np.ndarray]:
    """Oracle outputs of one case (keys prefixed `out_`)."""
    if name.startswith("q8_"):
        vocab, d = int(case["vocab"]), int(case["d"])
        ids = case["ids"].astype(np.int64)
        o0, _ = R.q8_0_embedding(case["blocks"], vocab, d, ids, act=0)
        o1, _ = R.q8_0_embedding(case["blocks"], vocab, d, ids, act=1)
        return {"out_none": o0, "out_silu": o1}
    if name.startswith("ln_c0"):
        return {"out_candle": R.layernorm_candle(case["x"], case["gamma"], case["beta"]),
                "out_twopass": R.layernorm_twopass(case["x"], case["gamma"], case["beta"])}
    if name.startswith("ln_unit_offset"):
        return {"out": R.layernorm_twopass(case["x"], case["gamma"], unit_offset=True)}
    if name.startswith("rope"):
        rot, theta, pos0 = int(case["rot"]), float(case["theta"]), int(case["pos0"])
        T = case["q"].shape[2]
        return {"out": R.rotary(case["q"], rot, theta, pos0), "table": R.rope_table(pos0 + T, rot, theta)}
    if name.startswith("adain"):
        f = lambda a: np.asarray(a).astype(np.float32)  # noqa: E731  (f16 params widen exactly)
        return {"out": R.adain_snake(case["x"], f(case["gamma"]), f(case["beta"]), f(case["alpha"]))}
    if name.startswith("resln_bf16"):
        wb = configs.f32_to_bf16_bits(case["gamma"])
        bb = configs.f32_to_bf16_bits(case["beta"])
        h, y = R.resadd_ln_gelu_bf16(case["x"], case["res"], wb, bb)
        return {"out_h": h, "out_y": y}
    if name.startswith("act"):
        return {"out_silu": R.silu(case["x"]), "out_gelu": R.gelu_erf(case["x"])}
    raise KeyError(name)


def build() -> None:
    for name, case in _inputs().items():
        case = dict(case)
        case.update(compute(name, case))
        np.savez_compressed(HERE / f"{name}.npz", **case)


def load_all() -> dict[str, dict[str, np.ndarray]]:
    out = {}
    for p in sorted(HERE.glob("*.npz")):
        with np.load(p, allow_pickle=False) as z:
            out[p.stem] = {k: z[k] for k in z.files}
    return out


if __name__ == "__main__":
    build()
    for p in sorted(HERE.glob("*.npz")):
        print(p.name, p.stat().st_size)
