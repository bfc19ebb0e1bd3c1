#!/usr/bin/env python3
"""Benchmark of the MI355X fused layer kernels (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workloads c1,c2,...] [--json-out FILE]

A step is one call of a fused kernel on one batch of synthetic input already
resident in HBM. The headline workload (`value`) is configs[4], the largest
configuration: AdaIN1d + Snake f32 x[8,128,115200] (workload c4b, the
dominant kernel by bytes), with configs[4]'s other kernel, residual add +
LayerNorm + GELU bf16 x,res [32,750,1024] (c4a), reported alongside in
`config`. Every other config (c0..c3) and the next-row workloads are
reported in `per_config`, one short array per workload (fields named by
`per_config_fields`). The line stays under 4 KB; the full record of every
workload (descriptions, kernels, warm and host figures, C++ enqueue times)
is printed to stderr as `[bench] full {...}` and written to --json-out.

Timing: input/output buffer sets rotate so the bytes touched between two
uses of a set are >= 512 MB (twice the 256 MB Infinity Cache): the timed
calls read HBM, not MALL. Before the timed region every set is run through
the kernel once (the touch pass, whose average is reported as
`first_touch_us_per_call`), then W untimed warm-up calls, then the K timed
calls continue the rotation. While the K calls are enqueued the stream is
held by a short spin kernel, so the GPU runs them back to back and the
timing is of the GPU, not the Python launch path. HIP events on the launch
stream bracket the K calls; `us_per_call` is their elapsed time / K, the
average launch duration. `warm_*` figures repeat one buffer set and are
labelled as such. `host_us_per_call` is the host time to enqueue one call
from Python (ctypes + the C-ABI runtime + hipModuleLaunchKernel);
`host_enqueue` is the same measured in C++ (nspeech_amd/host/
enqueue_bench.cpp) for the decode-step entry points, beside a bare
hipModuleLaunchKernel of an empty kernel, and per call of those entry
points captured for 24 decoder layers into one HIP graph and replayed
(`host_us_per_call_graph`). `spin_clock_MHz` is the shader clock the spin
kernel sees (its cycle counter per ms) at the start, after the MFMA conv
workloads and at the end.

Floors, measured in the same run through the same runtime: an empty kernel
(`empty`) and plain 128-bit device copies (`copy_<form>_<config>`) moving
exactly each config's algorithmic bytes (half read, half written), in two
grid forms (`f`: one 16-byte chunk per lane; `p4`/`p8`: a persistent
8 x #CU grid with 4 or 8 chunks per lane in flight). Each config's entry
carries `copy_floor_us` (the fastest copy of its size) and `frac_of_copy`.
rocprofv3's kernel trace adds about 3 us to kernels of a few us (it spaces
dispatches apart; the empty kernel shows 4.5 us there against 1.6 us back
to back); for the headline kernel its average over the timed calls agrees
with `us_per_call` to within 1% (profiles/bench_workloads_trace_and_traffic.md).
`traffic` is HBM bytes per dispatch from rocprofv3's FETCH_SIZE / WRITE_SIZE
counters, calibrated on the flat copy (profiles/hbm_traffic_bench_workloads.txt).

The CPU baseline is the oracle's C restatement of the reference CPU path
(oracle/nsr_oracle.c) timed on this host: per config the median of 20 runs
after 3 warm-ups, on 1 thread and on the host's threads, on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
CONFIG_WORKLOADS = ["c4b", "c4a", "c0", "c1", "c1t", "c2", "c3", "c2u", "c2h", "c4bh"]
NEXT_WORKLOADS = ["dec", "dec2", "attn", "attnx", "q8fc1", "q8fc2", "q8fc1r", "q8fc2r", "q8conv", "kconv3", "kconv7",
                  "kconv11", "kconv7f", "kconv11f", "kconv3u", "kchain3", "kchain11", "mrf", "istft"]
# same-size copies: algorithmic bytes of the config each one calibrates
COPY_SIZES = {"c1t": 8519680, "c3": 8642560, "c2h": 9833472, "c2": 19666944, "c4a": 196616192, "c4b": 943727104,
              "c4bh": 471863552}
COPY_FOR = {"c1": "c1t", "c1t": "c1t", "c3": "c3", "c2": "c2", "c2u": "c2", "c2h": "c2h", "c4a": "c4a", "c4b": "c4b",
            "c4bh": "c4bh", "c4a_act0": "c4a", "c4a_act1": "c4a"}
# c4bh gets the flat copy only: the persistent-grid forms were slower than it at every other size
FLOOR_WORKLOADS = ["empty"] + [f"copy_{f}_{c}" for c in COPY_SIZES for f in (("f",) if c == "c4bh" else ("f", "p4", "p8"))] \
    + ["copy_rows_c4b"]
DEFAULT_WORKLOADS = CONFIG_WORKLOADS + FLOOR_WORKLOADS + NEXT_WORKLOADS
MALL_DEFEAT_BYTES = 512 << 20
METRIC = "achieved HBM GB/s (% of MI355X peak) and µs/call per fused kernel"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workloads", default=",".join(DEFAULT_WORKLOADS),
                    help="comma list of " + ",".join(DEFAULT_WORKLOADS) + ",copy,c4a_act0,c4a_act1")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-rotate", action="store_true", help="one buffer set (warm MALL) for all timings")
    ap.add_argument("--no-touch-pass", action="store_true",
                    help="skip the pass that runs every buffer set once before the warm-up")
    ap.add_argument("--sets-on-held", action="store_true",
                    help="size the buffer-set rotation on the bytes a set holds, not the bytes a call touches "
                         "(for comparison: a partial gather then reuses sets within the Infinity Cache)")
    ap.add_argument("--fixed-hold", action="store_true",
                    help="hold the stream 5 ms + 0.1 ms per call before each timed run (the sizing before the hold "
                         "was fitted to the host's enqueue rate; an idle GPU before a burst slows the first "
                         "milliseconds of VALU-heavy work)")
    ap.add_argument("--json-out", default="", help="also write every workload's full record to this file")
    ap.add_argument("--timeline", action="store_true",
                    help="instead of the benchmark: the c4b call's timeline per workgroup and wave (one JSON line)")
    return ap.parse_args()


# ----------------------------------------------------------- workloads ---

class Workload:
    """Buffer sets and a launch(i) closure for one config.

    `set_bytes` is the memory one buffer set holds; `touched` the bytes one call
    reads or writes in it (less than `set_bytes` when a call reads a part of a
    table). The number of sets rotated is sized on the smaller of the two, so
    the bytes touched between two uses of a set exceed the Infinity Cache."""

    def __init__(self, name, desc, alg_bytes, set_bytes, make_set, launch, kernel, dtype, flops=0, touched=None):
        self.name, self.desc, self.alg_bytes = name, desc, alg_bytes
        self.set_bytes, self.make_set, self.launch = set_bytes, make_set, launch
        self.kernel, self.dtype, self.flops = kernel, dtype, flops
        self.touched = set_bytes if touched is None else touched


def build_workload(name):
    import numpy as np
    import torch

    from nspeech_amd import abi, configs

    L = abi.lib()
    dev = "cuda:0"
    stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    def T(a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint16:
            return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)
        if a.dtype == np.uint32:
            return torch.from_numpy(a.view(np.int32)).to(dev)
        return torch.from_numpy(a).to(dev)

    if name == "empty":
        def make_set(_):
            return {}

        def launch(s):
            abi.check(L.nsr_calib_empty(stream()))

        return Workload(name, "empty kernel (one launch on the stream)", 0, 1 << 30, make_set, launch,
                        "nsrk_calib_empty", "-")

    if name == "copy_rows_c4b":
        # c4b's bytes copied row by row (1024 rows of 115200 f32) with the AdaIN row kernel's access structure
        rows, rb = 1024, 115200 * 4

        def make_set(_):
            return {"s": torch.ones(rows * rb // 4, dtype=torch.float32, device=dev),
                    "d": torch.empty(rows * rb // 4, dtype=torch.float32, device=dev)}

        def launch(s):
            abi.check(L.nsr_calib_copy_rows(s["s"].data_ptr(), s["d"].data_ptr(), rows, rb, stream()))

        return Workload(name, f"row-by-row device copy of {rows} rows of {rb} bytes (the AdaIN row kernel's access "
                        "structure, one 512-lane workgroup per row)", 2 * rows * rb, 2 * rows * rb, make_set, launch,
                        "nsrk_calib_copy_rows", "u8")

    if name.startswith("copy_"):
        _, form, cfg = name.split("_")
        nbytes = COPY_SIZES[cfg] // 32 * 16  # half read, half written, in 16-byte chunks
        fi = {"f": 0, "p4": 1, "p8": 2}[form]

        def make_set(_):
            return {"s": torch.ones(nbytes // 4, dtype=torch.float32, device=dev),
                    "d": torch.empty(nbytes // 4, dtype=torch.float32, device=dev)}

        def launch(s):
            abi.check(L.nsr_calib_copy(s["s"].data_ptr(), s["d"].data_ptr(), nbytes, fi, 0, stream()))

        kern = {"f": "nsrk_calib_copy_flat", "p4": "nsrk_calib_copy_p4", "p8": "nsrk_calib_copy_p8"}[form]
        return Workload(name, f"device copy of {2 * nbytes} bytes ({nbytes} read + {nbytes} written), form {form} "
                        f"(the bytes of {cfg})", 2 * nbytes, 2 * nbytes, make_set, launch, kern, "u8")

    if name == "copy":
        n = 64 << 20  # 256 MiB of f32: plain device copy, the PMC calibration reference
        src = torch.ones(n, dtype=torch.float32, device=dev)

        def make_set(_):
            return {"o": torch.empty_like(src)}

        def launch(s):
            s["o"].copy_(src)

        return Workload(name, "plain device copy of 256 MiB (calibration)", 2 * n * 4, 2 * n * 4, make_set, launch,
                        "copy", "f32")

    if name == "c0":
        c = configs.c0()
        x0, g, b = T(c["x"]), T(c["gamma"]), T(c["beta"])

        def make_set(_):
            return {"x": x0.clone(), "y": torch.empty_like(x0)}

        def launch(s):
            abi.check(L.nsr_layernorm(s["x"].data_ptr(), 0, g.data_ptr(), b.data_ptr(), 0, s["y"].data_ptr(), 0,
                                      125, 1024, 1024, 1024, 1e-5, 0, 0, stream()))

        return Workload(name, "LayerNorm f32 x[1,125,1024] affine eps 1e-5", configs.algorithmic_bytes("c0"),
                        2 * 125 * 1024 * 4, make_set, launch, "nsrk_ln_f32_f32_nc4", "f32")

    if name in ("c1", "c1t"):
        c = configs.c1()
        q0, k0 = T(c["q"]), T(c["k"])
        table = abi.rope_table(1024, 32, 10000.0).to(dev) if name == "c1t" else None
        tp = table.data_ptr() if table is not None else None

        def make_set(_):
            return {"q": q0.clone(), "k": k0.clone(), "qo": torch.empty_like(q0), "ko": torch.empty_like(k0)}

        def launch(s):
            abi.check(L.nsr_rotary_partial_interleaved_f32(s["q"].data_ptr(), s["k"].data_ptr(), s["qo"].data_ptr(),
                                                           s["ko"].data_ptr(), 1, 8, 8, 1024, 64, 32, 10000.0, 0, tp,
                                                           1024 if tp else 0, stream()))

        extra = 1024 * 32 * 4 if name == "c1t" else 0
        return Workload(name, "partial interleaved rotary f32 q,k [1,8,1024,64] rot 32 theta 1e4"
                        + (" (host RoPE table)" if name == "c1t" else " (in-kernel sincos)"),
                        configs.algorithmic_bytes("c1") + extra, 4 * 8 * 1024 * 64 * 4, make_set, launch,
                        "nsrk_rope_table_f32" if name == "c1t" else "nsrk_rope_compute_f32", "f32")

    if name in ("c2", "c4b"):
        c = configs.c2() if name == "c2" else configs.c4b()
        x0 = T(c["x"])
        g, b, a = T(c["gamma"]), T(c["beta"]), T(c["alpha"])
        B, C, TT = c["x"].shape
        gs = C if c["gamma"].ndim == 2 else 0

        def make_set(_):
            return {"x": x0.clone() if name == "c2" else x0, "o": torch.empty_like(x0)}

        def launch(s):
            abi.check(L.nsr_adain_snake_f32(s["x"].data_ptr(), g.data_ptr(), b.data_ptr(), a.data_ptr(), 0, gs, gs,
                                            s["o"].data_ptr(), B, C, TT, 1e-5, stream()))

        kern = "nsrk_adain_row_b256_v5_l0" if name == "c2" else "nsrk_adain_row_b512_v38_l19"
        return Workload(name, f"AdaIN1d+Snake f32 x[{B},{C},{TT}]", configs.algorithmic_bytes(name),
                        2 * x0.numel() * 4, make_set, launch, kern, "f32")

    if name == "c2u":
        # c2 with an odd row length, as Kokoro's frame counts usually are: x f32 [1, 512, 4801] (rows not 16-byte
        # aligned, the unaligned resident kernel).
        c = configs.c2()
        g_ = configs.rng(1015)
        B, C, TT = 1, c["x"].shape[1], c["x"].shape[2] + 1
        x0 = T(g_.standard_normal((B, C, TT), dtype=np.float32))
        g, b, a = T(c["gamma"]), T(c["beta"]), T(c["alpha"])
        gs = C if c["gamma"].ndim == 2 else 0

        def make_set(_):
            return {"x": x0.clone(), "o": torch.empty_like(x0)}

        def launch(s):
            abi.check(L.nsr_adain_snake_f32(s["x"].data_ptr(), g.data_ptr(), b.data_ptr(), a.data_ptr(), 0, gs, gs,
                                            s["o"].data_ptr(), B, C, TT, 1e-5, stream()))

        alg = 4 * 2 * B * C * TT + 4 * 3 * C
        return Workload(name, f"AdaIN1d+Snake f32 x[{B},{C},{TT}] (unaligned rows)", alg, alg, make_set, launch,
                        "nsrk_adain_res_b256_nv5_u", "f32")

    if name == "c2h":
        # The c2 shape through the f16-activation entry point (the reference's KokoroGpuBackend::adain_snake,
        # whose Triton kernels take rows up to 8192): x, out f16 [1, 512, 4800], f16 style parameters.
        c = configs.c2()
        x0 = T(c["x"].astype(np.float16))
        g, b, a = (T(c[n].astype(np.float16)) for n in ("gamma", "beta", "alpha"))
        B, C, TT = c["x"].shape
        gs = C if c["gamma"].ndim == 2 else 0

        def make_set(_):
            return {"x": x0.clone(), "o": torch.empty_like(x0)}

        def launch(s):
            abi.check(L.nsr_adain_snake_f16(s["x"].data_ptr(), g.data_ptr(), b.data_ptr(), a.data_ptr(), 1, gs, gs,
                                            s["o"].data_ptr(), B, C, TT, 1e-5, stream()))

        alg = 2 * 2 * B * C * TT + 2 * 3 * C
        return Workload(name, f"AdaIN1d+Snake f16 activations x[{B},{C},{TT}]", alg, alg, make_set, launch,
                        "nsrk_adain_f16a_b256_nv3", "f16")

    if name == "c4bh":
        # configs[4]'s AdaIN shape through the f16-activation entry point (the reference's GPU backend runs the
        # Kokoro decoder in f16: KokoroGpuBackend::adain_snake): x, out f16 [8, 128, 115200], f16 parameters.
        c = configs.c4b()
        x0 = T(c["x"].astype(np.float16))
        g, b, a = (T(c[n].astype(np.float16)) for n in ("gamma", "beta", "alpha"))
        B, C, TT = c["x"].shape
        gs = C if c["gamma"].ndim == 2 else 0

        def make_set(_):
            return {"x": x0.clone(), "o": torch.empty_like(x0)}

        def launch(s):
            abi.check(L.nsr_adain_snake_f16(s["x"].data_ptr(), g.data_ptr(), b.data_ptr(), a.data_ptr(), 1, gs, gs,
                                            s["o"].data_ptr(), B, C, TT, 1e-5, stream()))

        alg = 2 * 2 * B * C * TT + 2 * (2 * B * C + C)
        return Workload(name, f"AdaIN1d+Snake f16 activations x[{B},{C},{TT}]", alg, 2 * x0.numel() * 2, make_set,
                        launch, "nsrk_adain_rowh_b512_v19_l10", "f16")

    if name == "c3":
        c = configs.c3()
        blocks0, ids = T(c["blocks"]), T(c["ids"])

        def make_set(_):
            return {"b": blocks0.clone(), "o": torch.empty((4096, 416), dtype=torch.float32, device=dev)}

        def launch(s):
            abi.check(L.nsr_q8_0_embed_gather(s["b"].data_ptr(), 32768, 416, ids.data_ptr(), 0, 4096,
                                              s["o"].data_ptr(), 1, None, stream()))

        # a call reads 4096 of the 32768 table rows: the sets are counted on the bytes touched, not held
        return Workload(name, "GGUF Q8_0 gather-dequant + SiLU, table 32768x416, 4096 ids -> f32 [4096,416]",
                        configs.algorithmic_bytes("c3"), blocks0.numel() + 4096 * 416 * 4, make_set, launch,
                        "nsrk_q8_0_gather_silu_u32", "i8xf16->f32", touched=configs.algorithmic_bytes("c3"))

    if name in ("dec", "dec2"):
        # Moonshine decoder step per layer (kernel_configs.py:102-104): q,k,v f16 [10, 64], rot 32,
        # caches [10, 448, 64]; "dec" = one launch, "dec2" = the reference's two dispatches
        # (rope_qk_cache_fused, then kv_cache_append).
        g = configs.rng(1006)
        Hq = Hk = 10
        Dh, rot, Lc, pos = 64, 32, 448, 300
        tab = abi.rope_table(Lc, rot, 10000.0).to(dev)
        mk = lambda *sh: torch.from_numpy(g.standard_normal(sh).astype(np.float16)).to(dev)  # noqa: E731

        def make_set(_):
            z = lambda: torch.zeros((Hk, Lc, Dh), dtype=torch.float16, device=dev)  # noqa: E731
            return {"q": mk(Hq, Dh), "k": mk(Hk, Dh), "v": mk(Hk, Dh), "ck": z(), "cv": z()}

        def launch(s):
            if name == "dec":
                abi.check(L.nsr_rope_qk_cache_append(s["q"].data_ptr(), s["k"].data_ptr(), s["v"].data_ptr(), 1,
                                                      tab.data_ptr(), Lc, s["ck"].data_ptr(), s["cv"].data_ptr(),
                                                      Hq, Hk, Dh, rot, pos, Lc, stream()))
            else:
                abi.check(L.nsr_rope_qk_cache_append(s["q"].data_ptr(), s["k"].data_ptr(), None, 1,
                                                      tab.data_ptr(), Lc, s["ck"].data_ptr(), None,
                                                      Hq, Hk, Dh, rot, pos, Lc, stream()))
                abi.check(L.nsr_kv_cache_append(s["v"].data_ptr(), s["cv"].data_ptr(), 1, Hk, Dh, Lc, pos,
                                                  stream()))

        alg = 2 * (2 * Hq * Dh + 2 * Hk * Dh) + 2 * (2 * Hk * Dh) + 2 * Hk * Dh + 4 * rot
        return Workload(name, "decode step RoPE(q,k) + K/V cache append f16, 10 heads x 64, rot 32"
                        + (" (one launch)" if name == "dec" else " (two launches, as the reference)"), alg,
                        2 * Hk * Lc * Dh * 2, make_set, launch,
                        "nsrk_rope_cache_f16", "f16")

    if name in ("attn", "attnx"):
        # Moonshine decoder attention at M = 1, 10 heads x 64, f16: "attn" = self-attention over the full KV
        # cache [10, 448, 64] (nsr_attention_decode_f16, split chosen by the library); "attnx" = cross-attention
        # over 30 s of encoder K/V [1500, 10, 64] with the reference's 32 splits (nsr_attention_splitkv_f16).
        g = configs.rng(1012)
        H, Dh = 10, 64
        kv_len = 448 if name == "attn" else 1500
        mk = lambda *sh: torch.from_numpy(g.standard_normal(sh).astype(np.float16)).to(dev)  # noqa: E731
        shape = (H, kv_len, Dh) if name == "attn" else (kv_len, H, Dh)
        skh, sks = (kv_len * Dh, Dh) if name == "attn" else (Dh, H * Dh)
        part = torch.empty(H * 32 * (Dh + 2), dtype=torch.float32, device=dev)

        def make_set(_):
            return {"q": mk(H, Dh), "k": mk(*shape), "v": mk(*shape), "o": torch.empty((H, Dh), dtype=torch.float16,
                                                                                      device=dev)}

        def launch(s):
            if name == "attn":
                abi.check(L.nsr_attention_decode_f16(s["q"].data_ptr(), s["k"].data_ptr(), s["v"].data_ptr(),
                                                     s["o"].data_ptr(), kv_len, Dh, H, H, 0.125, skh, sks, stream()))
            else:
                abi.check(L.nsr_attention_splitkv_f16(s["q"].data_ptr(), s["k"].data_ptr(), s["v"].data_ptr(),
                                                      s["o"].data_ptr(), part.data_ptr(), kv_len, Dh, H, H, 0.125,
                                                      skh, sks, 32, stream()))

        alg = 2 * (2 * H * Dh) + 2 * (2 * kv_len * H * Dh)
        return Workload(name, f"decode attention f16, 10 heads x 64, kv_len {kv_len}"
                        + (" (self-attention over the KV cache)" if name == "attn"
                           else " (cross-attention over the encoder K/V, 32 splits)"),
                        alg, alg, make_set, launch,
                        "nsrk_attn_head_d16" if name == "attn" else "nsrk_attn_partial_d16", "f16")

    if name in ("q8fc1", "q8fc2", "q8fc1r", "q8fc2r"):
        # Moonshine decoder MLP at M = 1 (dim 640, intermediate 2560; f16 activations, Q8 weights):
        # q8fc1 = fc1 + bias + GLU-SiLU (gemv_q8_bias_glu), q8fc2 = fc2 + residual + next LayerNorm
        # (gemv_q8_resadd_ln, two launches). q8fc1/q8fc2 read t4 tiles (nsr_q8_pack_t4, packed once per
        # buffer set outside the timed region); the "r" variants read the reference's [K, N/4] layout.
        # Every buffer set holds its own weight copy, so the timed calls stream the weights from HBM as a
        # decode step over many layers does.
        g = configs.rng(1007)
        dim, inter = 640, 2560
        fc1 = name.startswith("q8fc1")
        t4 = not name.endswith("r")
        K, NW = (dim, 2 * inter) if fc1 else (inter, dim)
        qs0 = torch.from_numpy(g.integers(0, 2 ** 32, size=(K, NW // 4), dtype=np.uint64).astype(np.uint32)
                               .view(np.int32)).to(dev)
        sc0 = torch.from_numpy((g.standard_normal((K // 32, NW)) * 0.02).astype(np.float16)).to(dev)
        x = torch.from_numpy(g.standard_normal(K).astype(np.float16)).to(dev)
        bias = torch.from_numpy(g.standard_normal(NW).astype(np.float32)).to(dev)
        res = torch.from_numpy(g.standard_normal(dim).astype(np.float32)).to(dev)
        lnw = torch.ones(dim, dtype=torch.float16, device=dev)

        def make_set(_):
            if t4:
                w = abi.Q8T4(qs0, sc0, glu=fc1)
                q, s_ = w.qs, w.scales
            else:
                q, s_ = qs0.clone(), sc0.clone()
            return {"q": q, "s": s_, "o": torch.empty(inter if fc1 else dim, dtype=torch.float16, device=dev),
                    "h": torch.empty(dim, dtype=torch.float32, device=dev)}

        f_glu = L.nsr_gemv_q8_t4_bias_glu if t4 else L.nsr_gemv_q8_bias_glu
        f_rln = L.nsr_gemv_q8_t4_resadd_ln if t4 else L.nsr_gemv_q8_resadd_ln

        def launch(s):
            if fc1:
                abi.check(f_glu(x.data_ptr(), 1, s["q"].data_ptr(), s["s"].data_ptr(), bias.data_ptr(),
                                s["o"].data_ptr(), 1, K, inter, stream()))
            else:
                abi.check(f_rln(x.data_ptr(), 1, s["q"].data_ptr(), s["s"].data_ptr(), res.data_ptr(),
                                s["h"].data_ptr(), lnw.data_ptr(), 1, s["o"].data_ptr(), 1, K, dim, 1e-5, stream()))

        wbytes = K * NW + (K // 32) * NW * 2
        lay = "t4 tiles" if t4 else "reference [K,N/4] layout"
        if fc1:
            alg = wbytes + 2 * K + 4 * NW + 2 * inter
            desc = f"Q8 GEMV fc1 + bias + GLU-SiLU, x f16 [{K}] @ W [{K},{NW}] ({lay}) -> f16 [{inter}]"
            kern = "nsrk_gemv_q8t4_glu_f16_f16_b256" if t4 else "nsrk_gemv_q8_glu_f16_f16"
        else:
            alg = wbytes + 2 * K + 4 * dim + 4 * dim + 2 * dim + 2 * dim
            desc = (f"Q8 GEMV fc2 + residual + LayerNorm, x f16 [{K}] @ W [{K},{NW}] ({lay}) -> f32 h, "
                    f"f16 norm [{dim}] (two launches)")
            kern = "nsrk_gemv_q8t4_h_f16_b1024" if t4 else "nsrk_gemv_q8_h_f16"
        return Workload(name, desc, alg, wbytes, make_set, launch, kern, "i8xf16->f32")

    if name == "q8conv":
        # Load-time conversion of a GGUF Q8_0 nn::Linear weight (the decoder fc1 [2*2560, 640] as the file
        # stores it: 5120 rows of 20 34-byte blocks) to t4 GLU tiles on the device (nsr_q8_0_to_t4): a byte
        # transpose, HBM-bound. Random block bytes stand in for the quantised weight (the kernel moves bytes).
        g = configs.rng(1008)
        N, K = 5120, 640
        src = torch.from_numpy(g.integers(0, 256, N * K // 32 * 34, dtype=np.uint8)).to(dev)

        def make_set(_):
            return {"b": src.clone(), "q": torch.empty(N * K // 4, dtype=torch.int32, device=dev),
                    "s": torch.empty(N * K // 32, dtype=torch.float16, device=dev)}

        def launch(s):
            abi.check(L.nsr_q8_0_to_t4(s["b"].data_ptr(), N, K, 1, s["q"].data_ptr(), s["s"].data_ptr(), stream()))

        alg = N * K // 32 * 34 + N * K + N * K // 32 * 2
        return Workload(name, f"GGUF Q8_0 weight [{N},{K}] -> t4 GLU tiles (load-time conversion)", alg, alg,
                        make_set, launch, "nsrk_gemv_q8_from_q8_0", "u8")

    if name == "mrf":
        # Kokoro multi-receptive-field average after the three resblocks of the last upsample stage, fused with the
        # leaky ReLU(0.01) before conv_post: ((r0 + r1) + r2) * f32(1/3), f32 [8, 128, 115200] (the c4b shape).
        B, C, TT = configs.c4b()["x"].shape
        g = configs.rng(1013)
        rs = [torch.from_numpy(g.standard_normal((B, C, TT), dtype=np.float32)).to(dev) for _ in range(3)]

        def make_set(_):
            return {"o": torch.empty_like(rs[0])}

        def launch(s):
            abi.check(L.nsr_resblock_average_f32(rs[0].data_ptr(), rs[1].data_ptr(), rs[2].data_ptr(),
                                                 s["o"].data_ptr(), B * C * TT, 1, 0.01, stream()))

        alg = 4 * 4 * B * C * TT
        return Workload(name, f"Kokoro MRF average + leaky ReLU f32 3 x [{B},{C},{TT}]", alg, alg, make_set, launch,
                        "nsrk_combine_f32_v", "f32")

    if name == "istft":
        # Kokoro iSTFT (n_fft 20, hop 5) of one utterance's conv_post output at the c4b frame count:
        # x f32 [22, 115200] (log-magnitudes, raw phases) -> 575995 samples (24 s at 24 kHz).
        n_frames, n_fft, hop = configs.c4b()["x"].shape[2], 20, 5
        g = configs.rng(1014)
        x0 = torch.from_numpy((g.standard_normal((2 * (n_fft // 2 + 1), n_frames)) * 0.7).astype(np.float32)).to(dev)
        out_len = (n_frames - 1) * hop

        def make_set(_):
            return {"x": x0.clone(), "o": torch.empty(out_len, dtype=torch.float32, device=dev)}

        def launch(s):
            abi.check(L.nsr_istft_f32(s["x"].data_ptr(), s["o"].data_ptr(), n_frames, out_len, n_fft, hop, stream()))

        alg = 4 * x0.numel() + 4 * out_len
        return Workload(name, f"Kokoro iSTFT n_fft {n_fft} hop {hop}, x f32 [22,{n_frames}] -> [{out_len}]", alg, alg,
                        make_set, launch, "nsrk_istft_f32_n20", "f32")

    if name in ("kconv3", "kconv7", "kconv11", "kconv3u", "kconv7f", "kconv11f"):
        # One Kokoro ResBlock stage at the final upsample shape (x [8, 128, 115200], as config c4b):
        # conv1(snake(AdaIN(x))) + bias at the Kokoro (K, dilation) pairs (3, 1), (7, 3), (11, 5), the workspace
        # offering the records part: from K = 7 the library takes the record path (row statistics, the records
        # pass with AdaIN + Snake, the MFMA kernel), below it the one-launch fused kernel (row statistics + the
        # conv with AdaIN + Snake in its producer waves). kconv7f / kconv11f = the one-launch kernels at K = 7 /
        # 11 (no records part); kconv3u = the K = 3 stage unfused (AdaIN+Snake kernel, then the one-launch conv).
        c = configs.c4b()
        x0 = T(c["x"])
        B, C, TT = c["x"].shape
        g_, b_, a_ = T(c["gamma"]), T(c["beta"]), T(c["alpha"])
        K, dil = {"kconv3": (3, 1), "kconv3u": (3, 1), "kconv7": (7, 3), "kconv7f": (7, 3), "kconv11": (11, 5),
                  "kconv11f": (11, 5)}[name]
        pad = (K - 1) * dil // 2
        g = configs.rng(1009)
        wp = abi.conv1d_pack_f16(torch.from_numpy((g.standard_normal((C, C, K)) * 0.05).astype(np.float16)).to(dev))
        bias = torch.from_numpy(g.standard_normal(C).astype(np.float16)).to(dev)
        gs = C if c["gamma"].ndim == 2 else 0
        y = torch.empty_like(x0) if name == "kconv3u" else None
        rec = name in ("kconv3", "kconv7", "kconv11")
        ws = abi.conv_workspace(B, C, C, TT, K, pad, dil, abi.WS_IN_STATS | (abi.WS_RECORDS if rec else 0), dev)

        def make_set(_):
            return {"x": x0, "o": torch.empty_like(x0)}

        def launch(s):
            if name == "kconv3u":
                abi.check(L.nsr_adain_snake_f32(s["x"].data_ptr(), g_.data_ptr(), b_.data_ptr(), a_.data_ptr(), 0, gs,
                                                gs, y.data_ptr(), B, C, TT, 1e-5, stream()))
                abi.check(L.nsr_conv1d_f16w_packed(y.data_ptr(), wp.data_ptr(), bias.data_ptr(), None,
                                                   s["o"].data_ptr(), B, C, C, TT, K, pad, dil, stream()))
            else:
                abi.check(L.nsr_adain_snake_conv1d_f32(s["x"].data_ptr(), g_.data_ptr(), b_.data_ptr(), a_.data_ptr(),
                                                       0, gs, gs, wp.data_ptr(), bias.data_ptr(), None,
                                                       s["o"].data_ptr(), B, C, C, TT, K, pad, dil, 1e-5,
                                                       ws.data_ptr(), ws.numel(), stream()))

        alg = 2 * x0.numel() * 4
        flops = 2 * C * C * K * TT * B
        return Workload(name, f"ResBlock stage AdaIN+Snake -> conv1d K={K} dil={dil} f32 x[{B},{C},{TT}]"
                        + {"kconv3u": " (unfused: two kernels + y round trip)", "kconv3": " (one-launch fused conv)",
                           "kconv7f": " (one-launch fused conv)", "kconv11f": " (one-launch fused conv)"}.get(
                            name, " (record path: statistics, records pass, MFMA kernel)"),
                        alg, x0.numel() * 4, make_set, launch,
                        {"kconv3": "nsrk_conv1d_rw_adain_snake_f16x2_nu3", "kconv7": "nsrk_conv1d_pr_f16x2",
                         "kconv11": "nsrk_conv1d_pr_f16x2", "kconv7f": "nsrk_conv1d_pc_adain_snake_f16x2_nu3",
                         "kconv11f": "nsrk_conv1d_pc_adain_snake_f16x2_nu4",
                         "kconv3u": "nsrk_conv1d_rw_f16x2_nu3"}[name], "f32",
                        flops=flops)

    if name in ("kchain3", "kchain11"):
        # The same ResBlock stage as kconv3 / kconv11 in the steady state of a chain: the input's row statistics
        # come from the previous stage (computed once, outside the timed calls) and the stage emits its output's
        # statistics for the next one (nsr_adain_snake_conv1d_chain_f32) instead of a separate statistics pass.
        c = configs.c4b()
        x0 = T(c["x"])
        B, C, TT = c["x"].shape
        g_, b_, a_ = T(c["gamma"]), T(c["beta"]), T(c["alpha"])
        K, dil = (11, 5) if name == "kchain11" else (3, 1)
        pad = (K - 1) * dil // 2
        g = configs.rng(1009)
        wp = abi.conv1d_pack_f16(torch.from_numpy((g.standard_normal((C, C, K)) * 0.05).astype(np.float16)).to(dev))
        bias = torch.from_numpy(g.standard_normal(C).astype(np.float16)).to(dev)
        gs = C if c["gamma"].ndim == 2 else 0
        xs = torch.empty((B * C, 2), dtype=torch.float32, device=dev)
        tmp = torch.empty_like(x0)
        ws = abi.conv_workspace(B, C, C, TT, K, pad, dil, abi.WS_OUT_STATS | abi.WS_RECORDS, dev)
        abi.check(L.nsr_conv1d_f16w_packed_stats(x0.data_ptr(), wp.data_ptr(), None, None, tmp.data_ptr(),
                                                 xs.data_ptr(), B, C, C, TT, K, pad, dil, 1e-5, ws.data_ptr(),
                                                 ws.numel(), stream()))
        # (statistics of some f32 [B, C, T] tensor; the timed calls use them for x, which only changes the values)
        del tmp

        def make_set(_):
            return {"x": x0, "o": torch.empty_like(x0), "s": torch.empty((B * C, 2), dtype=torch.float32,
                                                                          device=dev)}

        def launch(s):
            abi.check(L.nsr_adain_snake_conv1d_chain_f32(s["x"].data_ptr(), xs.data_ptr(), g_.data_ptr(),
                                                         b_.data_ptr(), a_.data_ptr(), 0, gs, gs, wp.data_ptr(),
                                                         bias.data_ptr(), None, s["o"].data_ptr(), s["s"].data_ptr(),
                                                         B, C, C, TT, K, pad, dil, 1e-5, ws.data_ptr(), ws.numel(),
                                                         stream()))

        alg = 2 * x0.numel() * 4
        flops = 2 * C * C * K * TT * B
        return Workload(name, f"ResBlock stage in a chain (statistics handed along) K={K} dil={dil} f32 x[{B},{C},{TT}]"
                        + (" (record path)" if K >= 7 else " (one-launch fused conv)"), alg, x0.numel() * 4, make_set,
                        launch, "nsrk_conv1d_pr_f16x2_st32" if K >= 7 else "nsrk_conv1d_rw_adain_snake_f16x2_nu3_st",
                        "f32", flops=flops)

    if name in ("c4a", "c4a_act0", "c4a_act1"):
        # c4a_act0 / c4a_act1: the same call without the activation / with SiLU (not default workloads: they
        # measure what the GELU epilogue costs)
        act = {"c4a": 2, "c4a_act0": 0, "c4a_act1": 1}[name]
        c = configs.c4a()
        x0, r0 = T(c["x"]), T(c["res"])
        g, b = T(c["gamma"]), T(c["beta"])

        def make_set(_):
            return {"x": x0.clone(), "r": r0.clone(), "h": torch.empty_like(x0), "y": torch.empty_like(x0)}

        def launch(s):
            abi.check(L.nsr_residual_add_layernorm(s["x"].data_ptr(), 2, s["r"].data_ptr(), 2, s["h"].data_ptr(), 2,
                                                   g.data_ptr(), b.data_ptr(), 0, s["y"].data_ptr(), 2, 24000, 1024,
                                                   1e-5, 0, act, stream()))

        return Workload(name, "residual add + LayerNorm + " + ["no activation", "SiLU", "GELU(erf)"][act]
                        + " bf16 x,res[32,750,1024] (writes h and y)",
                        configs.algorithmic_bytes("c4a"), 4 * x0.numel() * 2, make_set, launch,
                        "nsrk_resln_bf16_nc2", "bf16")
    raise KeyError(name)


def spin_rate_cycles_per_ms():
    import torch

    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(1000)
    s.record()
    torch.cuda._sleep(2_000_000)
    e.record()
    torch.cuda.synchronize()
    return 2_000_000 / max(s.elapsed_time(e), 1e-3)


def time_workload(w, steps, warmup, rotate, cyc_per_ms, touch_pass=True, sets_on_held=False, fixed_hold=False):
    """Time one workload. Order of GPU work: one untimed-for-the-headline
    call on every buffer set (the touch pass, so no timed call is the first
    kernel use of its buffers; its average is `first_touch_us_per_call`),
    `warmup` calls, then `steps` timed calls continuing the rotation where
    the warm-up stopped, so the bytes touched between two uses of a set stay
    above the Infinity Cache."""
    import torch

    per_set = w.set_bytes if sets_on_held else min(w.set_bytes, w.touched)
    nsets = max(1, math.ceil(MALL_DEFEAT_BYTES / per_set)) if rotate else 1
    sets = [w.make_set(i) for i in range(nsets)]
    torch.cuda.synchronize()

    host = []
    holds, attempts = [], []
    rate = {}  # host enqueue ms per call and GPU ms per call, from the touch pass

    def held(enqueue, n, hold_ms):
        """Hold the stream with a spin kernel for hold_ms while `enqueue`
        issues n calls, so the GPU then runs them back to back. Returns the
        host's enqueue time in ms."""
        torch.cuda.synchronize()
        torch.cuda._sleep(int(cyc_per_ms * hold_ms))
        h0 = time.perf_counter()
        enqueue()
        host_ms = (time.perf_counter() - h0) * 1e3
        torch.cuda.synchronize()
        host.append(host_ms * 1e3 / n)
        return host_ms

    def run_plain(order):
        """Time `order` back to back. The hold must let the host stay ahead of
        the GPU: call i is enqueued at about i * host rate and needed at
        hold + i * GPU rate, so the run is kept when the host finished within
        0.8 of (hold + the run's GPU time), else it is repeated with a longer
        hold. The first hold is fitted to the host rate of the warm-up (or the
        touch pass) and the GPU rate of the touch pass (0.5 ms + what the host
        needs beyond the GPU), so the GPU sits idle as briefly as the enqueue
        allows: an idle GPU slows the VALU-heavy work that follows it, from
        about the 40th call on and for longer than 200 calls (residual add +
        LayerNorm + GELU at [24000, 1024] bf16, 200 calls after 1 / 6 / 25 ms
        of idle: 33.5 / 34.3 / 34.7 us per call on MI355X). The touch pass,
        which has no rates yet, starts from 1 ms + 0.1 ms per call, and
        --fixed-hold from the earlier 5 ms + 0.1 ms per call everywhere."""
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = len(order)

        def enqueue():
            t0.record()
            for i in order:
                w.launch(sets[i])
            t1.record()

        base = 5.0 if fixed_hold else 1.0
        tries = [base + per_call * n for per_call in (0.1, 0.4, 1.6)]
        if rate and not fixed_hold:
            tries.insert(0, 0.5 + max(0.0, 1.25 * rate["host_ms"] * n - 0.8 * rate["gpu_ms"] * n))
        for k, hold_ms in enumerate(tries):
            host_ms = held(enqueue, n, hold_ms)
            gpu_ms = t0.elapsed_time(t1)
            if host_ms < 0.8 * (hold_ms + gpu_ms):
                break
        holds.append(round(hold_ms, 2))
        attempts.append(k + 1)
        return gpu_ms * 1e3 / n

    first_us = run_plain(list(range(nsets))) if touch_pass else None
    if touch_pass:
        rate.update(host_ms=host[-1] / 1e3, gpu_ms=first_us / 1e3)
    torch.cuda.synchronize()
    h0 = time.perf_counter()
    for i in range(warmup):
        w.launch(sets[i % nsets])
    if rate and warmup:  # the touch pass's few calls carry first-call host costs; the warm-up's rate is steadier
        rate["host_ms"] = min(rate["host_ms"], (time.perf_counter() - h0) * 1e3 / warmup)
    torch.cuda.synchronize()
    rotating = [(warmup + i) % nsets for i in range(steps)]
    cold_us = run_plain(rotating)            # timed region: K back-to-back calls
    warm_us = run_plain([0] * steps)         # same buffers: MALL-warm, labelled
    del sets
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    gbs = lambda us: w.alg_bytes / (us * 1e-6) / 1e9  # noqa: E731
    return {
        "workload": w.desc,
        "kernel": w.kernel,
        "dtype": w.dtype,
        "algorithmic_bytes": w.alg_bytes,
        "buffer_sets": nsets,
        "footprint_MB": round(nsets * w.set_bytes / 2**20, 1),
        "us_per_call": round(cold_us, 3),
        "GBs": round(gbs(cold_us), 1),
        "frac_of_peak": round(gbs(cold_us) / HBM_PEAK_GBS, 4),
        "first_touch_us_per_call": None if first_us is None else round(first_us, 3),
        "warm_us_per_call": round(warm_us, 3),
        "warm_GBs": round(gbs(warm_us), 1),
        **({"TFLOPs": round(w.flops / (cold_us * 1e-6) / 1e12, 2)} if w.flops else {}),
        "host_us_per_call": round(min(host), 2),
        "hold_ms": holds,
        "attempts": attempts,  # runs of the touch pass, the timed calls and the same-set calls (retries first)
    }


# ------------------------------------------------------------ timeline ---

def timeline_c4b(launches=20, reps=5):
    """--timeline: where a c4b call spends its time, per workgroup and wave.

    nsr_calib_adain_timeline is the c4b row kernel with s_memrealtime stamps (100 MHz) written from lane 0 of
    every wave: each workgroup's XCD and start, each wave's end and, per row, when the row's data had landed
    for the wave. Per rep, `launches` calls run back to back and the last one's stamps are read. Prints one
    JSON line (stdout): the workgroups' end times (from the first start) by XCD and over all, and within a
    workgroup how far apart its waves' row data landed. The output is checked against nsr_adain_snake_f32's."""
    import numpy as np
    import torch

    from nspeech_amd import abi, configs

    L = abi.lib()
    dev = "cuda:0"
    stream = torch.cuda.current_stream().cuda_stream
    c = configs.c4b()
    x, g, b, a = (torch.from_numpy(c[k]).to(dev) for k in ("x", "gamma", "beta", "alpha"))
    B, C, T = c["x"].shape
    out, ref = torch.empty_like(x), torch.empty_like(x)
    abi.check(L.nsr_adain_snake_f32(x.data_ptr(), g.data_ptr(), b.data_ptr(), a.data_ptr(), 0, C, C, ref.data_ptr(),
                                    B, C, T, 1e-5, stream))
    words = 80  # NSR_ADAIN_TL_WORDS
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    stamps = torch.zeros(4 * n_cu * words, dtype=torch.int64, device=dev)
    recs = []
    for _ in range(reps):
        stamps.zero_()
        torch.cuda.synchronize()
        for _ in range(launches):
            abi.check(L.nsr_calib_adain_timeline(x.data_ptr(), g.data_ptr(), b.data_ptr(), a.data_ptr(),
                                                 out.data_ptr(), B, C, T, stamps.data_ptr(), stamps.numel(),
                                                 stream))
        torch.cuda.synchronize()
        s = stamps.view(-1, words).cpu().numpy().astype(np.int64)
        s = s[s[:, 1] > 0]
        t0 = s[:, 1].min()
        end = (s[:, 2:10].max(axis=1) - t0) / 100.0
        xcc = s[:, 0]
        rows = -(-B * C // len(s))
        land = s[:, 10:10 + 8 * min(rows, 8)].reshape(len(s), -1, 8) / 100.0
        recs.append({"span_us": round(float(end.max()), 2),
                     "end_p10_median_max_us": [round(float(v), 2) for v in np.percentile(end, [10, 50, 100])],
                     "end_median_by_xcd_us": {int(k): round(float(np.median(end[xcc == k])), 2)
                                              for k in sorted(set(xcc.tolist()))},
                     "wave_landing_spread_median_us": round(float(np.median(land.max(2) - land.min(2))), 2)})
    line = {"timeline": "c4b AdaIN1d+Snake f32 x[8,128,115200], nsrk_adain_row_tl_b512_v38_l19",
            "workgroups": int(len(s)), "rows_per_workgroup": int(rows), "launches_per_rep": launches,
            "output_equals_adain_snake_f32": bool(torch.equal(out, ref)), "reps": recs}
    print(json.dumps(line), flush=True)


# -------------------------------------------------------- CPU baseline ---

def host_cpu():
    """(model name, threads used) of this host: the model from /proc/cpuinfo
    (what `lscpu` prints as "Model name"), the threads from the affinity mask,
    capped by OMP_NUM_THREADS when that is set (the GPU box's CPU share)."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return model, n


CPU_RUNS, CPU_WARMUPS = 20, 3


def cpu_baseline(names):
    """Oracle restatement of the reference CPU path, per config: the median of
    CPU_RUNS timed runs after CPU_WARMUPS untimed ones, on 1 thread and on the
    host's threads, each on a bounded sample of the config."""
    import numpy as np

    from nspeech_amd import configs
    from oracle import restated as R

    model, ncores = host_cpu()
    out = {}

    def timed(fn, alg_bytes):
        for _ in range(CPU_WARMUPS):
            fn()
        runs = []
        for _ in range(CPU_RUNS):
            t0 = time.perf_counter()
            fn()
            runs.append(time.perf_counter() - t0)
        us = float(np.median(runs)) * 1e6
        return {"us_per_call": round(us, 1), "GBs": round(alg_bytes / (us * 1e-6) / 1e9, 3), "calls": CPU_RUNS}

    for nm in names:
        if nm == "c1" or nm == "c1t":
            c = configs.c1()
            f1 = lambda: (R.rotary(c["q"], 32, 1e4, 0), R.rotary(c["k"], 32, 1e4, 0))  # noqa: E731
            fn = lambda: (R.rotary(c["q"], 32, 1e4, 0, nthreads=ncores), R.rotary(c["k"], 32, 1e4, 0,  # noqa: E731
                                                                                   nthreads=ncores))
            sample = "full config (q and k)"
        elif nm == "c0":
            c = configs.c0()
            f1 = lambda: R.layernorm_candle(c["x"], c["gamma"], c["beta"])  # noqa: E731
            fn = lambda: R.layernorm_candle(c["x"], c["gamma"], c["beta"], nthreads=ncores)  # noqa: E731
            sample = "full config"
        elif nm in ("c2", "c4b"):
            c = configs.c2() if nm == "c2" else configs.c4b(B=1, C=8)
            f1 = lambda: R.adain_snake(c["x"], c["gamma"], c["beta"], c["alpha"])  # noqa: E731
            fn = lambda: R.adain_snake(c["x"], c["gamma"], c["beta"], c["alpha"], nthreads=ncores)  # noqa: E731
            sample = "full config" if nm == "c2" else "8 of the 1024 rows (x[1,8,115200]), scaled"
        elif nm == "c3":
            c = configs.c3()
            ids = c["ids"].astype(np.int64)
            f1 = lambda: R.q8_0_embedding(c["blocks"], 32768, 416, ids, act=1)  # noqa: E731
            fn = None
            sample = "full config (whole-table dequantize, index_select, silu)"
        elif nm == "c4a":
            c = configs.c4a(rows=750)
            wb, bb = configs.f32_to_bf16_bits(c["gamma"]), configs.f32_to_bf16_bits(c["beta"])
            f1 = lambda: R.resadd_ln_gelu_bf16(c["x"], c["res"], wb, bb)  # noqa: E731
            fn = lambda: R.resadd_ln_gelu_bf16(c["x"], c["res"], wb, bb, nthreads=ncores)  # noqa: E731
            sample = "750 of the 24000 rows, scaled"
        elif nm in ("q8fc1", "q8fc2"):  # the "r" variants have the same CPU path
            g = configs.rng(1007)
            K, NW = (640, 5120) if nm.startswith("q8fc1") else (2560, 640)
            qs = g.integers(0, 2 ** 32, size=(K, NW // 4), dtype=np.uint64).astype(np.uint32)
            sc = (g.standard_normal((K // 32, NW)) * 0.02).astype(np.float16).view(np.uint16)
            xx = g.standard_normal(K).astype(np.float16).astype(np.float32)
            bb = g.standard_normal(NW).astype(np.float32)
            rr = g.standard_normal(640).astype(np.float32)
            ww = np.ones(640, np.float16).view(np.uint16)
            if nm.startswith("q8fc1"):
                f1 = lambda: R.gemv_q8(xx, qs, sc, bb, glu=True)  # noqa: E731
            else:
                f1 = lambda: R.gemv_q8_resadd_ln(xx, qs, sc, rr, ww)  # noqa: E731
            fn = None
            sample = "full config (scalar restatement of the Triton kernel, 1 thread)"
            wb = K * NW + (K // 32) * NW * 2
            galg = wb + 2 * K + (4 * NW + 2 * 2560 if nm.startswith("q8fc1") else 12 * 640)
            r1 = timed(f1, galg)
            out[nm] = {"sample": sample, "threads_1": {"us_per_call": r1["us_per_call"], "GBs": r1["GBs"]}}
            continue
        else:
            continue
        alg = configs.algorithmic_bytes("c1" if nm == "c1t" else nm)
        scale = {"c4b": 1024 // 8, "c4a": 24000 // 750}.get(nm, 1)
        r1 = timed(f1, alg / scale)
        entry = {"sample": sample, "threads_1": {"us_per_call": round(r1["us_per_call"] * scale, 1),
                                                 "GBs": r1["GBs"]}}
        if fn is not None:
            rn = timed(fn, alg / scale)
            entry[f"threads_{ncores}"] = {"us_per_call": round(rn["us_per_call"] * scale, 1), "GBs": rn["GBs"]}
        out[nm] = entry
    return out, ncores, model


# ----------------------------------------------------------------- main ---

# Fields of each workload in the stdout line's `per_config` (one array per workload). The full record of every
# workload (description, kernel, warm and host figures) goes to stderr and to --json-out.
PER_CONFIG_FIELDS = ["us_per_call", "GBs", "frac_of_peak", "copy_floor_us", "traffic", "first_touch_us_per_call"]
LINE_LIMIT_BYTES = 4096


def _finite(v):
    """JSON-safe number: None for NaN / inf (the stdout line stays strict JSON)."""
    if isinstance(v, float) and not math.isfinite(v):
        return None
    return v


def compact_line(results, steps, warmup, cpu, clocks):
    """The one stdout line: metric, value, the headline's roofline, the CPU
    baseline and one short array per workload. Kept under LINE_LIMIT_BYTES."""
    head_name = "c4b" if "c4b" in results else next(iter(results))
    head = results[head_name]
    companion = {}
    if "c4a" in results and head_name == "c4b":
        r = results["c4a"]
        companion = {"c4a": {"workload": "configs[4]: " + r["workload"], "kernel": r["kernel"], "dtype": r["dtype"],
                             "us_per_call": r["us_per_call"], "GBs": r["GBs"], "frac_of_peak": r["frac_of_peak"],
                             "copy_floor_us": r.get("copy_floor_us"), "traffic": r.get("traffic")}}
    per = {}
    for nm, r in results.items():
        if nm.startswith("copy_") and nm != "copy_rows_c4b":
            continue  # each copy is the copy_floor_us of its config
        per[nm] = [_finite(r.get(f)) for f in PER_CONFIG_FIELDS]
        if r.get("TFLOPs") is not None:
            per[nm].append(_finite(r["TFLOPs"]))
    line = {
        "metric": METRIC,
        "value": head["GBs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(head["us_per_call"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (seeded numpy inputs of the benchmark configs)",
        "config": {"workload": ("configs[4]: " if head_name == "c4b" else "") + head["workload"],
                   "buffer_sets": head["buffer_sets"], "footprint_MB": head["footprint_MB"],
                   "parallelism": "single GPU", **({"alongside": companion} if companion else {})},
        "roofline": {"bound": "hbm", "achieved": head["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": head["frac_of_peak"], "traffic": head.get("traffic"), "kernel": head["kernel"],
                     "us_per_call": head["us_per_call"], "copy_floor_us": head.get("copy_floor_us"),
                     "row_copy_floor_us": head.get("row_copy_floor_us")},
        "cpu_baseline": cpu,
        "spin_clock_MHz": clocks,
        "per_config_fields": PER_CONFIG_FIELDS + ["TFLOPs (MFMA workloads)"],
        "per_config": per,
    }
    return json.loads(json.dumps(line, allow_nan=False, default=_finite))


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs on a single MI355X (got --gpus {args.gpus}). "
              "The kernels shard with no exchange along rows/positions (one process per GPU, each on its own rows).",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from nspeech_amd import abi

    abi.init()
    if args.timeline:
        timeline_c4b()
        return
    names = [n for n in args.workloads.split(",") if n]
    # every workload's inputs are built before any is timed: the host takes up to seconds to generate the
    # larger ones, and an idle GPU slows the VALU-heavy work that follows it for longer than 200 calls
    # (the same idle-time effect the fitted hold avoids)
    built = {nm: build_workload(nm) for nm in names}
    print(f"[bench] built {len(built)} workloads", file=sys.stderr, flush=True)
    cyc = spin_rate_cycles_per_ms()
    # the spin kernel counts shader-clock cycles: its rate per ms is the clock of an idle-ish SIMD, taken before
    # the workloads, after the MFMA conv workloads and at the end
    clocks = {"start": round(cyc / 1e3)}
    mfma = [n for n in names if n.startswith(("kconv", "kchain"))]
    results = {}
    for nm in names:
        w = built.pop(nm)
        results[nm] = time_workload(w, args.steps, args.warmup, not args.no_rotate, cyc,
                                    touch_pass=not args.no_touch_pass, sets_on_held=args.sets_on_held,
                                    fixed_hold=args.fixed_hold)
        del w
        torch.cuda.empty_cache()
        print(f"[bench] {nm}: {results[nm]['us_per_call']} us/call, {results[nm]['GBs']} GB/s "
              f"({100 * results[nm]['frac_of_peak']:.1f}% of peak)", file=sys.stderr, flush=True)
        if mfma and nm == mfma[-1]:
            clocks["after_mfma"] = round(spin_rate_cycles_per_ms() / 1e3)
    clocks["end"] = round(spin_rate_cycles_per_ms() / 1e3)

    # host time per call of the decode-step entry points, measured in C++ (no binding overhead)
    host_enqueue = None
    eb = ROOT / "nspeech_amd" / "lib" / "nsr_enqueue_bench"
    if eb.exists():
        import subprocess

        # Under rocprofv3 (its settings reach the process as ROCPROF_* variables) the graph replay is left out:
        # a traced run ended in a segmentation fault inside hipGraphLaunch, which stays untraced.
        traced = any(k.startswith("ROCPROF_") for k in os.environ)
        r = subprocess.run([str(eb), str(eb.parent)] + (["--no-graph"] if traced else []),
                           capture_output=True, text=True, timeout=120)
        if r.returncode == 0 and r.stdout.strip():
            host_enqueue = json.loads(r.stdout.strip().splitlines()[-1])
            for nm in ("dec", "attn", "q8fc1"):
                if nm in results:
                    results[nm]["host_us_per_call_c"] = host_enqueue[nm]
                    # the same calls captured into one HIP graph (24 decoder layers) and replayed
                    if "graph_replay_per_call" in host_enqueue:
                        results[nm]["host_us_per_call_graph"] = host_enqueue["graph_replay_per_call"]
        else:
            print(f"[bench] enqueue bench failed ({r.returncode}): {r.stderr[-300:]}", file=sys.stderr, flush=True)

    # each config against the fastest same-size copy of this run
    for nm, r in results.items():
        cfg = COPY_FOR.get(nm)
        copies = [results[f"copy_{f}_{cfg}"]["us_per_call"] for f in ("f", "p4", "p8")
                  if f"copy_{f}_{cfg}" in results] if cfg else []
        if copies:
            r["copy_floor_us"] = min(copies)
            r["frac_of_copy"] = round(min(copies) / r["us_per_call"], 4)
        if nm == "c4b" and "copy_rows_c4b" in results:
            r["row_copy_floor_us"] = results["copy_rows_c4b"]["us_per_call"]
            r["frac_of_row_copy"] = round(r["row_copy_floor_us"] / r["us_per_call"], 4)

    traffic = {}
    tf = ROOT / "profiles" / "hbm_traffic_bench_workloads.txt"
    if tf.exists():
        for line in tf.read_text().splitlines():
            parts = line.split()  # workload kernel bytes
            if len(parts) == 3 and parts[2].isdigit() and parts[0] in results \
                    and results[parts[0]]["kernel"] == parts[1]:
                traffic[parts[0]] = int(parts[2])
    for nm, r in results.items():
        r["traffic"] = traffic.get(nm)

    cpu = None
    cpu_names = [n for n in names if n in CONFIG_WORKLOADS and n != "c1t"]
    if not args.no_cpu and cpu_names:
        per_cfg, ncores, model = cpu_baseline(cpu_names)
        head_name = "c4b" if "c4b" in per_cfg else next(iter(per_cfg))
        h = per_cfg[head_name]
        cpu = {"value": h["threads_1"]["GBs"], "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"oracle C restatement of the reference CPU path on {head_name}: {h['sample']}; median of "
                         f"{CPU_RUNS} runs after {CPU_WARMUPS} warm-ups, 1 thread",
               "cpu_model": model, "host_threads": ncores,
               "us_per_call": {nm: [e["threads_1"]["us_per_call"], e.get(f"threads_{ncores}", {}).get("us_per_call")]
                               for nm, e in per_cfg.items()},
               "us_per_call_fields": ["1 thread", f"{ncores} threads"]}
        print("[bench] cpu_baseline " + json.dumps(per_cfg), file=sys.stderr, flush=True)

    full = {"per_config": results, "host_enqueue": host_enqueue, "spin_clock_MHz": clocks}
    print("[bench] full " + json.dumps(full, default=_finite), file=sys.stderr, flush=True)
    if args.json_out:
        Path(args.json_out).parent.mkdir(parents=True, exist_ok=True)
        Path(args.json_out).write_text(json.dumps(full, indent=1, default=_finite) + "\n")
    line = compact_line(results, args.steps, args.warmup, cpu, clocks)
    sys.stderr.flush()
    print(json.dumps(line, allow_nan=False), flush=True)


if __name__ == "__main__":
    main()
