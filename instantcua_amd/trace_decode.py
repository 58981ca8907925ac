"""Stage timeline of the persistent decode kernel (a profiling tool, not part of the engine).

Loads ``libicua_trace.so`` (``python -m instantcua_amd.build --trace``), whose decode kernel
stamps the wall clock (100 MHz) at fixed points of every stage in the last step of a launch, and
prints a markdown table: for each point, when it is reached after the layer starts (the first
workgroup's QKV start), as the median over layers 4..23 of the median, earliest and latest
workgroup; then the same for the final norm, lm_head and the greedy commit.

Usage (on a GPU):  python -m instantcua_amd.trace_decode [--layers 28] [--pos 4096] [--steps 16] [--f16 | --q8]
                   python -m instantcua_amd.trace_decode --pairs   (a one-row and a grammar-pair pass)
The model is the 28-layer q4 group-64 decoder of the decode benchmark; the cache rows before
--pos are left zero (the bytes moved per step do not depend on their values).
"""
from __future__ import annotations

import argparse
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from instantcua_amd import engine as eng  # noqa: E402
from instantcua_amd import synth  # noqa: E402
from instantcua_amd.build import TRACE_LIB  # noqa: E402
from instantcua_amd.modelfile import WeightFormat  # noqa: E402

# Trace points of one layer, in stage order: (index in the kernel's trace row, who stamps it
# (math thread 0 or exchange thread 0), what has just happened).
LAYER_POINTS = [
    (0, "math", "layer start (QKV stage entered)"),
    (1, "exch", "x polled (QKV workgroups: 128..255; f16 / q8 all)"),
    (28, "math", "QKV matrix-core sums (before the reduction)"),
    (30, "math", "q|k|v published"),
    (2, "math", "K/V rows requested"),
    (3, "exch", "q|k|v of the group polled"),
    (21, "math", "attention operands built"),
    (25, "math", "K/V rows landed"),
    (27, "math", "scores and softmax done (last block)"),
    (29, "math", "P.V done"),
    (22, "math", "attention loop done"),
    (20, "math", "split partial published"),
    (5, "exch", "partials polled (mergers 224..255)"),
    (17, "math", "merge arithmetic done"),
    (6, "math", "merged heads published"),
    (7, "exch", "attention output polled (O workgroups 0..127)"),
    (8, "math", "O rows + residual published"),
    (9, "exch", "x' polled"),
    (13, "math", "x' staged (RMSNorm weights applied)"),
    (26, "math", "gate|up matrix-core sums (before the reduction)"),
    (14, "math", "gate|up matrix-core sums reduced"),
    (10, "math", "SwiGLU published"),
    (11, "exch", "h half polled"),
    (18, "math", "h staged"),
    (23, "math", "down half-block landed in LDS"),
    (24, "math", "down matrix-core sums"),
    (19, "math", "down reduced"),
    (12, "math", "down half published"),
]
HEAD_POINTS = [
    (0, "math", "lm_head stage entered"),
    (1, "exch", "final x polled"),
    (2, "math", "lm_head + workgroup argmax published"),
    (3, "exch", "256 argmax partials polled"),
    (4, "math", "token committed, next embedding built"),
]


def read_trace(layers: int, pos: int, steps: int, fmt: int = WeightFormat.Q4):
    eng.LIB_PATH = TRACE_LIB
    if not os.path.exists(TRACE_LIB):
        raise SystemExit(f"{TRACE_LIB} is missing: build it with python -m instantcua_amd.build --trace")
    if fmt == WeightFormat.F16:  # the f16 decode benchmark's model (random f16 bit patterns)
        img = synth.build_model_image(WeightFormat.F16, n_layers=layers, tag="bench-f16", f16_bits=True)
    elif fmt == WeightFormat.Q8:  # the q8 decode benchmark's model
        img = synth.build_model_image(WeightFormat.Q8, n_layers=layers, tag="bench-q8")
    else:
        img = synth.build_model_image(WeightFormat.Q4, n_layers=layers, tag="bench-q4")
    with eng.Engine(flags=0, image=img, max_context=pos + steps + 16, max_steps=steps + 8) as e:
        e.eos = (-1, -1)
        assert e.persistent_decode
        e.set_position(pos, 1234, 0, steps + 8)
        e.decode_steps(4)  # loads the code object; the next launch's last step is traced
        e.decode_steps(steps)
        us_tok = e.last_timing["decode_ms"] * 1e3 / steps
        buf = np.zeros((256, 29, 32), dtype=np.uint64)
        if eng.lib().icua_debug_persist_trace(buf.ctypes.data_as(C.c_void_p)) != 0:
            raise SystemExit("the loaded library has no trace")
    return buf.astype(np.float64) / 100.0, us_tok  # microseconds


def read_pair_traces(layers: int):
    """The last one-row pass and the last grammar-pair pass (two rows) of a greedy decode on the
    q4 decoder whose embedding rows of tokens 11 and 3678 are scaled by 8, so that pairs are
    forced; one decode_steps(1) call per pass.  [(name, trace, decode_steps ms), ...]."""
    eng.LIB_PATH = TRACE_LIB
    if not os.path.exists(TRACE_LIB):
        raise SystemExit(f"{TRACE_LIB} is missing: build it with python -m instantcua_amd.build --trace")
    img = synth.scale_embedding_rows(synth.build_model_image(WeightFormat.Q4, n_layers=layers, tag="bench-q4"),
                                     {11: 8.0, 3678: 8.0})
    toks = synth.random_tokens(9, "gram", 3)

    def grab():
        buf = np.zeros((256, 29, 32), dtype=np.uint64)
        if eng.lib().icua_debug_persist_trace(buf.ctypes.data_as(C.c_void_p)) != 0:
            raise SystemExit("the loaded library has no trace")
        return buf.astype(np.float64) / 100.0

    single = pair = None
    with eng.Engine(image=img, max_context=64, max_steps=40) as e:
        e.eos = (-1, -1)
        assert e.persistent_decode and e.grammar_pairs
        for _ in range(2):  # the first round loads the code objects
            e.prefill(toks, max_new=40)
            while not e.state()["done"]:
                was_pair = e.state()["n"] == 2
                e.decode_steps(1)
                got = (grab(), e.last_timing["decode_ms"])
                if was_pair:
                    pair = got
                elif not e.state()["done"]:  # a stopping pass leaves before the commit's last stamp
                    single = got
    if pair is None:
        raise SystemExit("no grammar pair was forced")
    return [("single-row pass", *single), ("pair pass", *pair)]


def table(t, layer_ids, points, title, x_pollers=slice(128, 256)):
    """x_pollers: the workgroups whose stamp 1 of a layer is the x poll (the others stamp their
    first barrier there): 128..255 in the q4 form, all 256 in the f16 / q8 form."""
    rows = [f"| {title} | stamped by | median WG (us) | earliest WG | latest WG |", "|---|---|---|---|---|"]
    for ev, who, what in points:
        med, lo, hi = [], [], []
        for l in layer_ids:
            start = np.min(t[:, l, 0][t[:, l, 0] > 0])
            v = t[x_pollers, l, ev] if (ev == 1 and points is LAYER_POINTS) else t[:, l, ev]
            v = v[v > 0] - start
            if v.size:
                med.append(np.median(v))
                lo.append(v.min())
                hi.append(v.max())
        if med:
            rows.append(f"| {what} | {who} | {np.median(med):.2f} | {np.median(lo):.2f} | {np.median(hi):.2f} |")
    return "\n".join(rows)


WG_CLASSES = [("0..127", slice(0, 128)), ("128..223", slice(128, 224)), ("224..255", slice(224, 256))]


def class_table(t, layer_ids, points, title):
    """Median and latest stamp of each workgroup class (0..127: O and the lower down halves;
    128..255: QKV; 224..255 also merge), median over the layers; "-" where a class never stamps."""
    head = " | ".join(f"{n} median | {n} latest" for n, _ in WG_CLASSES)
    rows = [f"| {title} | {head} |", "|---|" + "---:|" * (2 * len(WG_CLASSES))]
    for ev, _, what in points:
        cells = []
        for _, sl in WG_CLASSES:
            med, hi = [], []
            for l in layer_ids:
                start = np.min(t[:, l, 0][t[:, l, 0] > 0])
                v = t[sl, l, ev]
                v = v[v > 0] - start
                if v.size:
                    med.append(np.median(v))
                    hi.append(v.max())
            cells += [f"{np.median(med):.2f}", f"{np.median(hi):.2f}"] if med else ["-", "-"]
        rows.append(f"| {what} | " + " | ".join(cells) + " |")
    return "\n".join(rows)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--pos", type=int, default=4096)
    ap.add_argument("--steps", type=int, default=16)
    ap.add_argument("--f16", action="store_true", help="the 28-layer f16 decoder instead of q4")
    ap.add_argument("--q8", action="store_true", help="the 28-layer q8 g32 decoder instead of q4")
    ap.add_argument("--classes", action="store_true", help="also tabulate each workgroup class's median and latest stamps")
    ap.add_argument("--save", default=None, help="write the raw stamp array [workgroup][layer][event] (us) to this .npy file")
    ap.add_argument("--pairs", action="store_true",
                    help="tabulate a one-row pass and a grammar-pair pass of the pair-forcing model instead")
    a = ap.parse_args()
    if a.pairs:
        for name, t, ms in read_pair_traces(a.layers):
            starts = [np.min(t[:, l, 0][t[:, l, 0] > 0]) for l in range(a.layers + 1)]
            print(f"## {name}: decode_steps(1) {ms * 1e3:.1f} us; layer period median "
                  f"{np.median(np.diff(starts[:a.layers])[4:24]):.2f} us; lm_head+commit "
                  f"{np.max(t[:, a.layers, 4]) - starts[a.layers]:.2f} us\n")
            print(table(t, list(range(4, 24)), LAYER_POINTS, "layer point"))
            print()
        return
    fmt = WeightFormat.F16 if a.f16 else WeightFormat.Q8 if a.q8 else WeightFormat.Q4
    name = "f16" if a.f16 else "q8" if a.q8 else "q4"
    t, us_tok = read_trace(a.layers, a.pos, a.steps, fmt)
    L = a.layers
    starts = [np.min(t[:, l, 0][t[:, l, 0] > 0]) for l in range(L + 1)]
    period = np.diff(starts[:L])
    mid = list(range(min(4, L - 1), max(min(24, L - 1), 5)))
    print(f"Persistent decode, {L}-layer {name} decoder, context {a.pos}, {a.steps} steps in one launch: "
          f"{us_tok:.1f} us/token with the trace stores (the last step is traced).\n")
    print(f"Layer period (layer start to the next layer's start): median {np.median(period[mid[0]:mid[-1]]):.2f} us, "
          f"min {period.min():.2f}, max {period.max():.2f}; final norm + lm_head + commit "
          f"{np.max(t[:, L, 4]) - starts[L]:.2f} us.\n")
    print(table(t, mid, LAYER_POINTS, f"layer point (median of layers {mid[0]}..{mid[-1]})",
                slice(0, 256) if fmt != WeightFormat.Q4 else slice(128, 256)))
    print()
    print(table(t, [L], HEAD_POINTS, "lm_head / commit point"))
    if a.classes:
        print()
        print(class_table(t, mid, LAYER_POINTS, "layer point, by workgroup class"))
    if a.save:
        np.save(a.save, t)


if __name__ == "__main__":
    main()
