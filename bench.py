#!/usr/bin/env python3
"""Fresh-encode benchmark on one MI355X.

Workload (BASELINE.json ``configs[1]``, "C2"): the Qwen3-8B tokenizer, one
fresh request of 4,194,304 characters from the seeded Zipf token-concat
generator, mixed script (85% ASCII words, 10% Latin-1 accented words, 5%
whitespace runs with tabs and CR LF). A step is one encode of one request.

``value`` is the whole-job throughput in millions of characters per second
with the UTF-8 bytes already resident in HBM (``tk_engine_encode_device``:
every kernel, the count read-back and the id copy, until the ids are
final). Each of the K timed steps encodes a different request (windows of
one seeded stream), and every step's ids are checked bit for bit against
the CPU oracle after the timed region. The PCIe-inclusive latency (host
UTF-8 in, host uint32 ids out, ``tk_engine_encode``) is reported beside it.

Also on the JSON line:
- ``roofline``: the dominant kernel's (k_bpe_pack, the packed merge)
  achieved bandwidth, taken as the per-request algorithmic bytes (UTF-8
  bytes read once + 4 bytes per id written once) over its average duration
  in the timed region, from the pair of HIP events its own dispatch takes
  on the engine's stream (timing mode 2: one timed dispatch per request),
  against the 8 TB/s HBM peak. ``traffic`` is the kernel's measured HBM
  bytes per launch from the committed rocprofv3 counter summary
  (profiles/c<config>_traffic.json) when it was taken on the library build
  being run, else null.
- ``stage_us``: per-stage device times from a second, untimed pass over the
  same requests with an event on every stage boundary (timing mode 1; those
  events add a few microseconds each, so that pass is not the timed one).
- ``cpu_baseline``: the C restatement (oracle) timed on this host's cores
  on a bounded sample of the same workload, one thread.

``--gpus N`` with N > 1 exits: this build runs on one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = ("4M-char fresh-encode latency (ms) + Mchars/s, HBM GB/s % peak; "
          "bit-exact IDs")
HBM_PEAK_GBS = 8000.0
TARGET_MS = 3.88


def pct(xs, q):
    return float(np.percentile(np.asarray(xs), q))


def measured_traffic(config: int, kernel: str):
    """HBM bytes per launch of `kernel` (FETCH_SIZE + WRITE_SIZE, scaled by
    a plain copy's reading) from the committed rocprofv3 summary, when that
    summary was taken on a library built from these very sources, flags and
    compiler (the manifest's build key); else None."""
    try:
        with open(os.path.join(ROOT, "profiles", f"c{config}_traffic.json")) as f:
            d = json.load(f)
        with open(os.path.join(ROOT, "toktier_amd", "_lib", "manifest.json")) as f:
            m = json.load(f)
    except (OSError, ValueError):
        return None
    if d.get("build_key") != m.get("build_key") or d.get("kernel") != kernel:
        return None
    return int(d["fetch_bytes"] + d["write_bytes"])


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2, choices=[2, 4, 5])
    ap.add_argument("--family", default=None,
                    help="encode the config's text with another family "
                         "(e.g. laguna_s_2_1 on C4's code-like stream)")
    ap.add_argument("--chat", action="store_true",
                    help="lay the config's text out as chat turns in the "
                         "family's template (added-token literals, split "
                         "out on the device)")
    ap.add_argument("--seed", action="store_true",
                    help="time the session seed instead (tk_engine_encode_seed: "
                         "ids plus span checkpoints every 4096 tokens), a "
                         "second workload line, not the contract line")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline leg")
    ap.add_argument("--no-check", action="store_true",
                    help="skip the per-step oracle parity check")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 10 plain device-to-device copies of MIB "
                         "MiB (the reference kernel for scaling the "
                         "FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        n = args.copy_calibration << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 10}))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on exactly one GPU; "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2
    K, W = max(1, args.steps), max(0, args.warmup)

    import torch
    import toktier_amd
    from toktier_amd import workloads

    fam, gen = workloads.CONFIGS[args.config]
    if args.family:
        fam = args.family
    if args.chat:
        gen = lambda js, n_chars: workloads.chat(js, fam, n_chars=n_chars)  # noqa: E731
    tok = toktier_amd.load(fam)
    eng = tok.engine
    n_chars = workloads.CHARS_4M
    log = lambda *a: print(*a, file=sys.stderr, flush=True)  # noqa: E731

    # K + W distinct requests: windows of one seeded stream
    t0 = time.perf_counter()
    n_req = K + W
    stream_text = gen(tok._json, n_chars=n_chars + 64 * n_req)
    reqs = []
    for i in range(n_req):
        off = (i * 64) % (len(stream_text) - n_chars + 1)
        reqs.append(stream_text[off:off + n_chars].encode("utf-8"))
    log(f"generated {n_req} requests in {time.perf_counter() - t0:.1f}s")

    dev = torch.device("cuda:0")
    d_texts = [torch.frombuffer(bytearray(r), dtype=torch.uint8).to(dev)
               for r in reqs]
    cap = max(len(r) for r in reqs)
    # one id buffer per request: the ids are copied out after the timed
    # region, so the steps run back to back
    d_ids = [torch.empty(cap, dtype=torch.int32, device=dev)
             for _ in range(n_req)]
    torch.cuda.synchronize()
    eng.set_timing(2)  # k_bpe_pack's own dispatch only

    stride = toktier_amd.SPAN_CHECKPOINT_STRIDE
    n_pts = cap // stride + 1
    d_pts = ([torch.empty(3 * n_pts, dtype=torch.int64, device=dev)
              for _ in range(n_req)] if args.seed else [])

    def run(i):
        d = d_texts[i]
        if args.seed:
            return eng.encode_seed(d.data_ptr(), d.numel(), d_ids[i].data_ptr(),
                                   cap, stride, d_pts[i].data_ptr(), n_pts)[0]
        return eng.encode_device(d.data_ptr(), d.numel(), d_ids[i].data_ptr(),
                                 cap)

    for i in range(W):
        run(K + i)
    torch.cuda.synchronize()
    lat, pack_us, n_ids = [], [], []
    t_all = time.perf_counter()
    for i in range(K):
        t1 = time.perf_counter()
        n_ids.append(run(i))
        lat.append((time.perf_counter() - t1) * 1e3)
        pack_us.append(eng.last_timing()[1])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_all
    ms_per_step = float(np.mean(lat))
    ids_dev = [d_ids[i][:n_ids[i]].cpu().numpy().view(np.uint32).copy()
               for i in range(K)]

    # per-stage breakdown: the same requests again, events on every stage
    eng.set_timing(1)
    stages = []
    for i in range(K):
        if run(i) != ids_dev[i].size:
            log(f"stage pass: id count differs on request {i}")
            return 1
        stages.append(eng.last_timing())
    eng.set_timing(0)

    # PCIe-inclusive: host bytes in -> host ids out
    host_lat = []
    for i in range(K):
        t1 = time.perf_counter()
        out = eng.encode(reqs[i])
        host_lat.append((time.perf_counter() - t1) * 1e3)
        if not np.array_equal(out, ids_dev[i]):
            log(f"host/device id mismatch on request {i}")
            return 1

    # parity: every timed request against the oracle
    mism = 0
    if not args.no_check:
        from oracle.oracle import Oracle
        from toktier_amd import classes
        f = tok.family
        orc = Oracle(tok.tables, classes.table_for(tok.family.ruleset_name), classes.nfc_qc_table(),
                     f.ruleset, f.digits_max, f.needs_nfc)
        orc.set_added([t.content.encode() for t in tok.added_tokens],
                      [t.id for t in tok.added_tokens])
        for i in range(K):
            want = orc.encode_bytes(reqs[i])
            if isinstance(want, int) or not np.array_equal(want, ids_dev[i]):
                mism += 1
        log(f"parity: {K - mism}/{K} requests bit-identical to the oracle")
        if args.seed:
            # the checkpoints of two requests against the store's restated
            # construction over the oracle's ids
            from oracle.oracle import span_checkpoints, token_byte_lengths
            lens = token_byte_lengths(tok._json)
            for t in tok.added_tokens:
                lens[t.id] = len(t.content.encode("utf-8"))
            for i in range(min(K, 2)):
                m = (ids_dev[i].size + stride - 1) // stride
                got = d_pts[i][:3 * m].cpu().numpy().view(np.uint64).reshape(m, 3)
                want = span_checkpoints(reqs[i], ids_dev[i], lens, stride)
                if not np.array_equal(got, want):
                    mism += 1
                    log(f"seed checkpoints differ on request {i}")

    n_tok = float(np.mean([a.size for a in ids_dev]))
    n_bytes = float(np.mean([len(r) for r in reqs[:K]]))
    st = np.asarray(stages)  # [K, 5]: pretok, bpe_small, bpe_long, compact, total
    names = ["pretokenize + piece lists (k_pretok, k_lists, k_pack_copy)",
             "k_bpe_pack",
             "long pieces past k_bpe_pack (k_bpe_rows, k_bpe_wide, k_long_*, "
             "k_certify; side stream)",
             "compaction (k_compact)"]
    avg = st[:, :4].mean(axis=0)
    pack_avg_us = float(np.mean(pack_us))
    b_alg = n_bytes + 4.0 * n_tok
    achieved = b_alg / (pack_avg_us * 1e-6) / 1e9

    cpu = None
    if not args.no_cpu:
        from oracle.oracle import Oracle
        from toktier_amd import classes
        f = tok.family
        orc = Oracle(tok.tables, classes.table_for(tok.family.ruleset_name), classes.nfc_qc_table(),
                     f.ruleset, f.digits_max, f.needs_nfc)
        orc.set_added([t.content.encode() for t in tok.added_tokens],
                      [t.id for t in tok.added_tokens])
        t1 = time.perf_counter()
        done = 0
        chars = 0
        while done < len(reqs) and (time.perf_counter() - t1) < 12.0:
            orc.encode_bytes(reqs[done])
            chars += n_chars
            done += 1
        dt = time.perf_counter() - t1
        cpu = {"value": round(chars / dt / 1e6, 3), "unit": "Mchars/s",
               "cores": 1, "kind": "port",
               "sample": f"{done} x {n_chars}-char requests of the same "
                         "workload through the C restatement (oracle/), "
                         "one thread, this host",
               "ms_per_request": round(dt / done * 1e3, 2)}

    line = {
        "metric": METRIC,
        "value": round(n_chars / (ms_per_step * 1e-3) / 1e6, 2),
        "unit": "Mchars/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic: seeded Zipf token-concat generator over the "
                "stand-in vocabulary of the family",
        "config": {
            "workload": f"C{args.config}{' chat' if args.chat else ''}"
                        f"{' seed' if args.seed else ''}: "
                        f"{fam}, one fresh request of {n_chars:,} chars"
                        f"{' in chat turns (added-token literals)' if args.chat else ''}"
                        ", bytes resident in HBM"
                        f"{'; ids plus span checkpoints every 4096 tokens (tk_engine_encode_seed)' if args.seed else ''}",
            "family": fam, "chars": n_chars, "bytes": int(n_bytes),
            "tokens": int(n_tok), "requests": K,
        },
        "latency_ms": {"p50": round(pct(lat, 50), 4),
                       "p90": round(pct(lat, 90), 4),
                       "p99": round(pct(lat, 99), 4)},
        "host_latency_ms": {"p50": round(pct(host_lat, 50), 4),
                            "p90": round(pct(host_lat, 90), 4),
                            "p99": round(pct(host_lat, 99), 4),
                            "note": "PCIe-inclusive: host UTF-8 in, host ids out"},
        "target_ms": TARGET_MS,
        "tokens_per_s": round(n_tok / (ms_per_step * 1e-3), 1),
        "stage_us": {n: round(float(v), 2) for n, v in zip(names, avg)},
        "roofline": {
            "bound": "hbm",
            "kernel": "k_bpe_pack",
            "kernel_us": round(pack_avg_us, 2),
            "achieved": round(achieved, 3),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 6),
            "traffic": (None if args.chat or args.family or args.seed else
                        measured_traffic(args.config, "k_bpe_pack")),
            "alg_bytes_per_launch": int(b_alg),
            "path_achieved": round(b_alg / (ms_per_step * 1e-3) / 1e9, 3),
        },
        "cpu_baseline": cpu,
        "parity": {"checked": 0 if args.no_check else K, "mismatches": mism},
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)
    tok.close()
    return 0 if mism == 0 else 1


if __name__ == "__main__":
    sys.exit(main())
