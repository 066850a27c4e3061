#!/usr/bin/env python3
"""Fresh-encode benchmark on one MI355X.

Workload (BASELINE.json ``configs[1]``, "C2"): the Qwen3-8B tokenizer, one
fresh request of 4,194,304 characters from the seeded Zipf token-concat
generator, mixed script (85% ASCII words, 10% Latin-1 accented words, 5%
whitespace runs with tabs and CR LF). A step is one encode of one request.
``--config 4`` / ``--config 5`` run C4 (Llama-3, code-like) / C5 (Qwen3,
CJK / emoji with ten 65,536-char letter runs) the same way; ``--config 3``
runs C3 (GPT-2, a ragged batch of 256 requests) as one batch per step.

Every step is a DISTINCT seeded request (``workloads.configN(sample=i)``,
generated in a process pool before the GPU is touched), and every step's
ids are checked bit for bit against the CPU oracle after the timed region.

``value`` / ``ms_per_step``: whole-job throughput (million characters per
second) and mean latency with the UTF-8 bytes already resident in HBM
(``tk_engine_encode_device``: every kernel and the count read-back, until
the ids are final in device memory). For C3, which the engine takes only
from host memory (``tk_engine_encode_batch_docs``: each document in its own
buffer, as the reference's ``texts: &[&str]``), they are the host-to-host
batch figures, ids into a reused page-locked buffer.

``protocol``: the reference's timing window (host UTF-8 buffer in, host
``uint32`` ids out, transfers included; ``tk_engine_encode``), p50 / p90 /
p99 over the same distinct requests after warm-ups, with chars/s and
tokens/s. The 3.88 ms bar (``target_ms``) is quoted on this window.

Also on the JSON line:
- ``roofline``: the dominant kernel's achieved bandwidth, taken as the
  per-request algorithmic bytes (UTF-8 bytes read once + 4 bytes per id
  written once) over its average duration in the timed region. The
  dominant kernel is the one with the largest median own duration in an
  untimed stage pass over the timed requests, with every kernel timed on
  its own dispatch (timing mode 1); the timed loop then times that
  kernel's dispatch alone, with
  the pair of HIP events it takes on the stream it runs on (timing mode 2,
  ``TK_OPT_TIMED_KERNEL``). Against the 8 TB/s HBM peak. ``traffic`` is
  its measured HBM bytes per launch from the committed rocprofv3 counter
  summary (profiles/c<config>_traffic.json) when that was taken on the
  library build being run and on the same kernel, else null.
- ``stage_us`` / ``kernels_us``: per-stage device times and every kernel's
  own mean duration from a second, untimed pass over the same requests
  (timing mode 1; those events add a few microseconds each, so that pass
  is not the timed one).
- ``other_configs`` (the default C2 run only; ``--no-legs`` skips it): C3,
  C4 and C5 with ``--leg-steps`` distinct requests each: protocol p50 /
  p90 / p99, the device-resident time, parity against the oracle, the
  dominant kernel and its roofline fraction, each kernel's duration.
- ``cpu_baseline``: the C restatement (oracle) timed on this host's cores on
  a bounded sample of the same workload, on every core the process may use
  (one request per thread); ``cpu_lanes`` adds the same on one core and
  HF ``tokenizers`` (the engine every id is certified against) pinned to
  one core with ``RAYON_NUM_THREADS=1`` (C3: ``encode_batch`` on one core
  and on all cores), each on distinct requests, with the host's facts
  (``nproc``, CPU model, affinity).

``--gpus N`` with N > 1 exits: this build runs on one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = ("4M-char fresh-encode latency (ms) + Mchars/s, HBM GB/s % peak; "
          "bit-exact IDs")
HBM_PEAK_GBS = 8000.0
TARGET_MS = 3.88
MAX_WORKERS = 16  # the GPU box's CPU share


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def pct(xs, q):
    return float(np.percentile(np.asarray(xs), q))


def pcts(xs, nd=4):
    return {"p50": round(pct(xs, 50), nd), "p90": round(pct(xs, 90), nd),
            "p99": round(pct(xs, 99), nd)}


def host_facts() -> dict:
    aff = sorted(os.sched_getaffinity(0))
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True,
                             timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    if model is None:
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    return {"nproc": os.cpu_count(), "cpu_model": model,
            "affinity": len(aff), "affinity_cpus": aff[:64]}


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


# ------------------------------------------------------------ requests

def _gen(job):
    """One request of the workload (a worker of the generation pool): the
    UTF-8 bytes, or for C3 the list of documents' bytes."""
    config, fam, chat, sample, n_chars = job
    from toktier_amd import standin, workloads
    js = standin.load_artifact_json(fam)
    if config == 3:
        return [d.encode("utf-8") for d in workloads.config3(js, sample=sample)]
    if chat:
        return workloads.chat(js, fam, n_chars=n_chars,
                              sample=sample).encode("utf-8")
    gen = workloads.CONFIGS[config][1]
    return gen(js, n_chars=n_chars, sample=sample).encode("utf-8")


def make_requests(config, fam, chat, n, n_chars, first_sample=1,
                  max_workers=MAX_WORKERS):
    """n distinct seeded requests (samples first_sample .. first_sample+n-1),
    generated in parallel before anything touches the GPU."""
    import multiprocessing as mp
    jobs = [(config, fam, chat, first_sample + i, n_chars) for i in range(n)]
    workers = max(1, min(max_workers, len(os.sched_getaffinity(0)), n))
    if workers == 1:
        return [_gen(j) for j in jobs]
    with mp.get_context("fork").Pool(workers) as pool:
        return pool.map(_gen, jobs)


def n_chars_of(req) -> int:
    if isinstance(req, list):
        return sum(len(d.decode("utf-8")) for d in req)
    return len(req.decode("utf-8"))


# ------------------------------------------------------------ CPU lanes

def make_oracle(tok):
    from oracle.oracle import Oracle
    from toktier_amd import classes
    from toktier_amd import families
    f = tok.family
    orc = Oracle(tok.tables, classes.table_named(families.class_table_name(f)),
                 classes.nfc_qc_table(), f.ruleset, f.digits_max, f.needs_nfc,
                 contractions=f.contractions)
    orc.set_added([t.content.encode() for t in tok.added_tokens],
                  [t.id for t in tok.added_tokens])
    return orc


def oracle_lane(orc, reqs, threads: int, budget_s: float) -> dict:
    """The oracle (one request per thread at a time; the C calls release
    the GIL) over as many of `reqs` as fit the time budget."""
    from concurrent.futures import ThreadPoolExecutor
    docs = []
    for r in reqs:
        docs.extend(r if isinstance(r, list) else [r])
    # the oracle keeps no cache, so the sample cycles through the requests
    # until the budget is spent
    import itertools
    t0 = time.perf_counter()
    done_bytes = done_chars = done = 0
    lat = []
    with ThreadPoolExecutor(threads) as ex:
        it = itertools.cycle(docs)
        while time.perf_counter() - t0 < budget_s:
            batch = [d for _, d in zip(range(threads), it)]

            def one(d):
                t1 = time.perf_counter()
                orc.encode_bytes(d)
                return time.perf_counter() - t1
            lat.extend(ex.map(one, batch))
            done += len(batch)
            done_bytes += sum(len(d) for d in batch)
            done_chars += sum(len(d.decode("utf-8")) for d in batch)
    dt = time.perf_counter() - t0
    return {"value": round(done_chars / dt / 1e6, 3), "unit": "Mchars/s",
            "cores": threads, "requests": done, "bytes": done_bytes,
            "seconds": round(dt, 2),
            "ms_per_request_p50": round(pct(lat, 50) * 1e3, 2) if lat else None}


_HF_CHILD = r"""
import json, os, sys, time
cpus = json.loads(sys.argv[3])
os.sched_setaffinity(0, cpus)
from tokenizers import Tokenizer
tok = Tokenizer.from_file(sys.argv[1])
reqs = json.load(open(sys.argv[2]))
budget = float(sys.argv[4]); batch = sys.argv[5] == "1"
t0 = time.perf_counter(); lat = []; chars = 0; n = 0
for r in reqs:
    if time.perf_counter() - t0 > budget and n > 0:
        break
    t1 = time.perf_counter()
    if batch:
        tok.encode_batch(r, add_special_tokens=False)
        chars += sum(len(d) for d in r)
    else:
        tok.encode(r, add_special_tokens=False)
        chars += len(r)
    lat.append(time.perf_counter() - t1); n += 1
dt = time.perf_counter() - t0
print(json.dumps({"chars": chars, "seconds": dt, "requests": n, "lat": lat}))
"""


def hf_lane(tokenizer_json: str, reqs, cpus: list[int], budget_s: float,
            batch: bool) -> dict | None:
    """HF tokenizers in a child process pinned to `cpus` (rayon threads =
    len(cpus)), over distinct requests until the budget is spent."""
    with tempfile.TemporaryDirectory() as d:
        tj = os.path.join(d, "tokenizer.json")
        with open(tj, "w", encoding="utf-8") as f:
            f.write(tokenizer_json)
        rj = os.path.join(d, "reqs.json")
        # HF keeps a word cache: every sample is a distinct request (a few
        # fill the budget at about a second each)
        reqs = reqs[:8]
        if batch:
            payload = [[x.decode("utf-8") for x in r] for r in reqs]
        else:
            payload = [r.decode("utf-8") for r in reqs]
        with open(rj, "w", encoding="utf-8") as f:
            json.dump(payload, f)
        env = dict(os.environ, RAYON_NUM_THREADS=str(len(cpus)),
                   TOKENIZERS_PARALLELISM="true" if len(cpus) > 1 else "false")
        try:
            res = subprocess.run(
                [sys.executable, "-c", _HF_CHILD, tj, rj, json.dumps(cpus),
                 str(budget_s), "1" if batch else "0"],
                capture_output=True, text=True, env=env,
                timeout=budget_s * 4 + 120)
        except subprocess.TimeoutExpired:
            return None
    if res.returncode != 0:
        log("HF lane failed:", res.stderr[-500:])
        return None
    r = json.loads(res.stdout.strip().splitlines()[-1])
    return {"value": round(r["chars"] / r["seconds"] / 1e6, 3),
            "unit": "Mchars/s", "cores": len(cpus), "requests": r["requests"],
            "seconds": round(r["seconds"], 2),
            "ms_per_request_p50": round(pct(r["lat"], 50) * 1e3, 2),
            "engine": "HF tokenizers " + _hf_version()}


def _hf_version() -> str:
    try:
        import tokenizers
        return tokenizers.__version__
    except Exception:
        return "?"


def cpu_lanes(tok, config: int, reqs, budget_s: float) -> tuple[dict, dict]:
    aff = sorted(os.sched_getaffinity(0))[:MAX_WORKERS]
    orc = make_oracle(tok)
    lanes = {"host": host_facts()}
    log(f"cpu lanes: oracle on 1 core, {len(aff)} cores; HF pinned")
    lanes["oracle_1core"] = oracle_lane(orc, reqs, 1, budget_s)
    lanes["oracle_ncores"] = oracle_lane(orc, reqs, len(aff), budget_s)
    if config == 3:
        lanes["hf_1core"] = hf_lane(tok._json, reqs, aff[:1], budget_s, True)
        lanes["hf_ncores"] = hf_lane(tok._json, reqs, aff, budget_s, True)
    else:
        lanes["hf_1core"] = hf_lane(tok._json, reqs, aff[:1], budget_s, False)
    lanes["reference_published"] = {
        "hf_tokenizers_1core_4MB_p50_ms": 1250.985,
        "toktier_cpu_gigatoken_1core_4MB_p50_ms": 8.817,
        "source": "docs/benchmarks.md:25-26, :77, :85 (2x EPYC 9115)"}
    o = lanes["oracle_ncores"]
    base = {"value": o["value"], "unit": "Mchars/s", "cores": o["cores"],
            "kind": "port",
            "sample": f"{o['requests']} distinct requests of the same workload "
                      f"through the C restatement (oracle/), one request per "
                      f"thread on {o['cores']} cores of this host, "
                      f"{o['seconds']} s"}
    return base, lanes


# ------------------------------------------------------------ measurement

def kernel_names():
    from toktier_amd._ffi import KERNELS
    return KERNELS


def kernel_pass(eng, run, idxs):
    """Timing mode 1 over the requests `idxs` (untimed: every kernel's own
    dispatch carries an event pair, which delays the next dispatch by a few
    microseconds): per request the stage times [0..4] and each kernel's own
    duration (0 when the call did not launch it)."""
    names = kernel_names()
    eng.set_timing(1)
    st, ku = [], []
    for i in idxs:
        run(i)
        t = eng.last_timing()
        st.append(t[:5])
        ku.append(t[8:8 + len(names)])
    eng.set_timing(0)
    return np.asarray(st), np.asarray(ku)


def dominant_kernel(ku) -> int:
    """The kernel with the largest median own duration per request."""
    return int(np.argmax(np.median(np.asarray(ku), axis=0)))


def launch_mean(xs) -> float:
    """Mean duration over the requests that launched the kernel."""
    xs = [x for x in xs if x > 0]
    return float(np.mean(xs)) if xs else 0.0


def roofline(kernel: str, kernel_us: float, b_alg: float, traffic) -> dict:
    achieved = b_alg / (kernel_us * 1e-6) / 1e9 if kernel_us > 0 else 0.0
    return {"bound": "hbm", "kernel": kernel, "kernel_us": round(kernel_us, 2),
            "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 6), "traffic": traffic,
            "alg_bytes_per_launch": int(b_alg)}


def measure_single(tok, reqs, K, W, seed=False, plain=True):
    """Requests 0..K-1 timed, K..K+W-1 warm-ups. After the warm-ups, an
    untimed stage pass over the timed requests with every kernel timed
    (mode 1) names the dominant kernel (largest median own duration); the
    timed loop (device-resident: bytes in HBM, ids compacted into a device
    buffer) times that kernel's own dispatch only (mode 2); then the
    protocol window (host UTF-8 in, host uint32 ids out) over the same
    requests."""
    import torch
    import toktier_amd
    from toktier_amd import _ffi
    eng = tok.engine
    dev = torch.device("cuda:0")
    d_texts = [torch.frombuffer(bytearray(r), dtype=torch.uint8).to(dev)
               for r in reqs]
    cap = max(len(r) for r in reqs)
    d_ids = [torch.empty(cap, dtype=torch.int32, device=dev)
             for _ in range(K + W)]
    stride = toktier_amd.SPAN_CHECKPOINT_STRIDE
    n_pts = cap // stride + 1
    d_pts = ([torch.empty(3 * n_pts, dtype=torch.int64, device=dev)
              for _ in range(K + W)] if seed else [])
    torch.cuda.synchronize()

    def run(i):
        d = d_texts[i]
        if seed:
            return eng.encode_seed(d.data_ptr(), d.numel(), d_ids[i].data_ptr(),
                                   cap, stride, d_pts[i].data_ptr(), n_pts)[0]
        return eng.encode_device(d.data_ptr(), d.numel(), d_ids[i].data_ptr(), cap)

    for i in range(K, K + W):
        run(i)
    stages, ku = kernel_pass(eng, run, range(K))
    kdom = dominant_kernel(ku)
    eng.set_option(_ffi.TK_OPT_TIMED_KERNEL, kdom)
    eng.set_timing(2)
    torch.cuda.synchronize()
    lat, kus, n_ids = [], [], []
    t_all = time.perf_counter()
    for i in range(K):
        t1 = time.perf_counter()
        n_ids.append(run(i))
        lat.append((time.perf_counter() - t1) * 1e3)
        kus.append(eng.last_timing()[1])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_all
    eng.set_timing(0)
    ids_dev = [d_ids[i][:n_ids[i]].cpu().numpy().view(np.uint32).copy()
               for i in range(K)]

    # the protocol window, into a reused numpy id buffer as a serving loop
    # keeps one: page-locked (the compaction kernel writes the ids straight
    # into it) and plain pageable memory (through the engine's pinned
    # staging); the request bytes are ordinary Python bytes either way
    out_pinned = torch.empty(cap + 1, dtype=torch.int32,
                             pin_memory=True).numpy().view(np.uint32)
    out_plain = np.zeros(cap + 1, dtype=np.uint32)

    def protocol(out):
        for i in range(K, K + W):
            eng.encode(reqs[i], out=out)
        lat_, parts_, ok_ = [], [], True
        for i in range(K):
            t1 = time.perf_counter()
            got = eng.encode(reqs[i], out=out)
            lat_.append((time.perf_counter() - t1) * 1e3)
            parts_.append(eng.last_timing()[5:8])
            if not np.array_equal(got, ids_dev[i]):
                log(f"host/device id mismatch on request {i}")
                ok_ = False
        return lat_, parts_, ok_
    host_lat, host_parts, ok1 = protocol(out_pinned)
    plain_lat, plain_parts, ok2 = protocol(out_plain) if plain else ([], [], True)
    return {"lat": lat, "wall": wall, "kernel": kdom, "kernel_us": kus,
            "ids": ids_dev, "stages": stages, "ku": ku,
            "host_lat": host_lat, "host_parts": host_parts,
            "plain_lat": plain_lat, "plain_parts": plain_parts,
            "host_ok": ok1 and ok2, "d_pts": d_pts, "stride": stride}


def measure_batch(tok, reqs, K, W):
    """C3: a ragged batch per step through tk_engine_encode_batch_docs (host
    documents in, each in its own buffer; host ids, into a reused
    page-locked buffer as a serving loop keeps one, and row offsets out). An untimed stage pass
    (mode 1) names the dominant kernel; the timed loop times its dispatch
    (mode 2). Here k_compact writes the ids straight into page-locked host
    memory, so its duration includes that PCIe write."""
    import torch
    from toktier_amd import _ffi
    eng = tok.engine
    cap = max(sum(len(d) for d in r) for r in reqs) + 1
    out = torch.empty(cap, dtype=torch.int32, pin_memory=True).numpy().view(np.uint32)

    def run(i):
        return eng.encode_batch(reqs[i], out=out)
    for i in range(K, K + W):
        run(i)
    stages, ku = kernel_pass(eng, run, range(K))
    kdom = dominant_kernel(ku)
    eng.set_option(_ffi.TK_OPT_TIMED_KERNEL, kdom)
    eng.set_timing(2)
    lat, rows_all, kus = [], [], []
    t_all = time.perf_counter()
    for i in range(K):
        t1 = time.perf_counter()
        ids, rows, status = run(i)
        lat.append((time.perf_counter() - t1) * 1e3)
        kus.append(eng.last_timing()[1])
        rows_all.append((ids[:int(rows[-1])].copy(), rows.copy(), status.copy()))
    wall = time.perf_counter() - t_all
    eng.set_timing(0)
    return {"lat": lat, "wall": wall, "kernel": kdom, "kernel_us": kus,
            "rows": rows_all, "stages": stages, "ku": ku}


def check_parity(tok, reqs, ids) -> int:
    """Every request against the oracle (threads: the C calls release the
    GIL); returns the number of mismatching requests."""
    from concurrent.futures import ThreadPoolExecutor
    orc = make_oracle(tok)

    def one(i):
        want = orc.encode_bytes(reqs[i])
        return not (isinstance(want, int) or not np.array_equal(want, ids[i]))
    n = max(1, min(MAX_WORKERS, len(os.sched_getaffinity(0))))
    with ThreadPoolExecutor(n) as ex:
        ok = list(ex.map(one, range(len(reqs))))
    mism = len(ok) - sum(ok)
    log(f"parity: {sum(ok)}/{len(ok)} requests bit-identical to the oracle")
    return mism


def check_batch_parity(tok, reqs, rows_all) -> int:
    """Every row of every batch against the oracle's encode of that
    document alone; returns the number of batches with a mismatching row."""
    from concurrent.futures import ThreadPoolExecutor
    orc = make_oracle(tok)

    def one(i):
        ids, rows, status = rows_all[i]
        for d, doc in enumerate(reqs[i]):
            want = orc.encode_bytes(doc)
            got = ids[int(rows[d]):int(rows[d + 1])]
            if status[d] != 0 or isinstance(want, int) or not np.array_equal(got, want):
                return 1
        return 0
    n = max(1, min(MAX_WORKERS, len(os.sched_getaffinity(0))))
    with ThreadPoolExecutor(n) as ex:
        bad = list(ex.map(one, range(len(rows_all))))
    log(f"parity: {len(bad) - sum(bad)}/{len(bad)} batches with every row "
        f"bit-identical to the oracle")
    return sum(bad)


def check_seed(tok, reqs, ids_dev, d_pts, stride, K) -> int:
    """The checkpoints of two requests against the store's restated
    construction over the engine's ids."""
    from oracle.oracle import span_checkpoints, token_byte_lengths
    lens = token_byte_lengths(tok._json)
    for t in tok.added_tokens:
        lens[t.id] = len(t.content.encode("utf-8"))
    mism = 0
    for i in range(min(K, 2)):
        m = (ids_dev[i].size + stride - 1) // stride
        got = d_pts[i][:3 * m].cpu().numpy().view(np.uint64).reshape(m, 3)
        want = span_checkpoints(reqs[i], ids_dev[i], lens, stride)
        if not np.array_equal(got, want):
            mism += 1
            log(f"seed checkpoints differ on request {i}")
    return mism


STAGE_NAMES = ["pretokenize and piece lists (k_added, k_pretok)",
               "k_bpe_pack",
               "long pieces past k_bpe_pack (k_bpe_rows, k_bpe_wide, k_long_*, "
               "k_certify; side streams)",
               "compaction (k_compact)"]


def kernel_summary(ku) -> dict:
    """Each kernel's mean own duration (us) over the requests that
    launched it, from the stage pass."""
    names = kernel_names()
    ku = np.asarray(ku)
    return {n: round(launch_mean(ku[:, k]), 2) for k, n in enumerate(names)
            if (ku[:, k] > 0).any()}


LEG_WORKLOADS = {
    3: "C3: GPT-2, a ragged batch of 256 requests of U[1,024, 32,768] chars "
       "(host documents in, host ids and row offsets out)",
    4: "C4: Llama-3, one 4,194,304-char code-like request",
    5: "C5: Qwen3, one 4,194,304-char request, 50% CJK, 10% emoji, ten "
       "65,536-char letter runs",
}


def leg(config: int, K: int, W: int, gen_workers: int) -> dict:
    """A compact line for another configuration: protocol latency, the
    device-resident time, parity against the oracle, the dominant kernel
    and its roofline fraction."""
    import toktier_amd
    from toktier_amd import workloads
    fam = workloads.CONFIGS[config][0]
    t0 = time.perf_counter()
    reqs = make_requests(config, fam, False, K + W, workloads.CHARS_4M,
                         max_workers=gen_workers)
    log(f"leg C{config}: {K + W} requests in {time.perf_counter() - t0:.1f}s")
    import torch  # noqa: F401
    tok = toktier_amd.load(fam)
    names = kernel_names()
    try:
        if config == 3:
            m = measure_batch(tok, reqs, K, W)
            mism = check_batch_parity(tok, reqs[:K], m["rows"])
            n_tok = float(np.mean([r[0].size for r in m["rows"]]))
            n_bytes = float(np.mean([sum(len(d) for d in r) for r in reqs[:K]]))
            host = m["lat"]
            dev_ms = None
        else:
            m = measure_single(tok, reqs, K, W, plain=False)
            mism = check_parity(tok, reqs[:K], m["ids"]) + (0 if m["host_ok"] else 1)
            n_tok = float(np.mean([a.size for a in m["ids"]]))
            n_bytes = float(np.mean([len(r) for r in reqs[:K]]))
            host = m["host_lat"]
            dev_ms = pcts(m["lat"])
        chars = float(np.mean([n_chars_of(r) for r in reqs[:K]]))
        kname = names[m["kernel"]]
        out = {
            "workload": LEG_WORKLOADS[config],
            "family": fam, "requests": K, "warmup": W, "chars": int(chars),
            "bytes": int(n_bytes), "tokens": int(n_tok),
            "protocol_latency_ms": pcts(host),
            "protocol_mchars_per_s": round(chars / (np.mean(host) * 1e-3) / 1e6, 2),
            "device_resident_latency_ms": dev_ms,
            "roofline": roofline(kname, launch_mean(m["kernel_us"]),
                                 n_bytes + 4.0 * n_tok,
                                 measured_traffic(config, kname)),
            "kernels_us": kernel_summary(m["ku"]),
            "parity": {"checked": K, "mismatches": mism,
                       "against": "CPU oracle" + (", every row" if config == 3 else "")},
        }
    finally:
        tok.close()
    return out


# ------------------------------------------------------------ main

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2, choices=[2, 3, 4, 5])
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
                    help="skip the CPU baseline lanes")
    ap.add_argument("--no-legs", action="store_true",
                    help="skip the C3 / C4 / C5 legs of the default run")
    ap.add_argument("--leg-steps", type=int, default=8,
                    help="requests per C3 / C4 / C5 leg")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="time budget of each CPU lane")
    ap.add_argument("--no-check", action="store_true",
                    help="skip the per-step oracle parity check")
    ap.add_argument("--gen-workers", type=int, default=MAX_WORKERS,
                    help="processes generating the requests (1 under a "
                         "profiler that loads itself into every process)")
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
    if args.config == 3 and (args.seed or args.chat):
        print("bench.py: --config 3 is a batch; --seed / --chat do not apply",
              file=sys.stderr)
        return 2

    from toktier_amd import workloads
    fam = args.family or workloads.CONFIGS[args.config][0]
    n_chars = workloads.CHARS_4M

    # K + W distinct seeded requests, before the GPU is touched
    t0 = time.perf_counter()
    reqs = make_requests(args.config, fam, args.chat, K + W, n_chars,
                         max_workers=args.gen_workers)
    log(f"generated {K + W} distinct requests in {time.perf_counter() - t0:.1f}s")
    batch = args.config == 3

    # the CPU lanes, also before the GPU is touched (their child processes
    # are started from a process that has not initialised it)
    cpu, lanes = None, None
    import toktier_amd
    if not args.no_cpu:
        from toktier_amd import bpe_tables, families, standin  # noqa: F401

        class _Tok:  # what the lanes need of a Tokenizer, without a device
            pass
        t = _Tok()
        t._json = standin.load_artifact_json(fam)
        t.tables = bpe_tables.load_tables(t._json)
        t.family = families.family(fam)
        t.added_tokens = toktier_amd.added_tokens(t._json)
        cpu, lanes = cpu_lanes(t, args.config, reqs, args.cpu_seconds)

    import torch  # noqa: F401  (before the engine opens: torch's HIP init first)
    tok = toktier_amd.load(fam)
    names = kernel_names()
    plain_traffic = not (args.chat or args.family or args.seed)
    if batch:
        m = measure_batch(tok, reqs, K, W)
        mism = 0 if args.no_check else check_batch_parity(tok, reqs[:K], m["rows"])
        n_tok = float(np.mean([r[0].size for r in m["rows"]]))
        n_bytes = float(np.mean([sum(len(d) for d in r) for r in reqs[:K]]))
        ms = float(np.mean(m["lat"]))
        host_lat = m["lat"]
    else:
        m = measure_single(tok, reqs, K, W, seed=args.seed)
        mism = 0 if m["host_ok"] else 1
        if not args.no_check:
            mism += check_parity(tok, reqs[:K], m["ids"])
            if args.seed:
                mism += check_seed(tok, reqs, m["ids"], m["d_pts"], m["stride"], K)
        n_tok = float(np.mean([a.size for a in m["ids"]]))
        n_bytes = float(np.mean([len(r) for r in reqs[:K]]))
        ms = float(np.mean(m["lat"]))
        host_lat = m["host_lat"]
    chars = float(np.mean([n_chars_of(r) for r in reqs[:K]]))
    b_alg = n_bytes + 4.0 * n_tok
    kname = names[m["kernel"]]
    host_ms = float(np.mean(host_lat))
    st = np.asarray(m["stages"])
    if batch:
        workload = (f"C3: {fam}, a ragged batch of 256 requests of U[1,024, "
                    "32,768] chars per step, host documents in, host ids and "
                    "row offsets out (tk_engine_encode_batch_docs; the engine "
                    "takes batches from host memory only, so value is "
                    "host-to-host)")
    else:
        workload = (f"C{args.config}{' chat' if args.chat else ''}"
                    f"{' seed' if args.seed else ''}: {fam}, one fresh request "
                    f"of {n_chars:,} chars"
                    f"{' in chat turns (added-token literals)' if args.chat else ''}"
                    ", bytes resident in HBM"
                    f"{'; ids plus span checkpoints every 4096 tokens (tk_engine_encode_seed)' if args.seed else ''}")
    protocol = {
        "window": ("host UTF-8 buffer in -> host uint32 ids out "
                   "(tk_engine_encode, transfers included); request bytes in "
                   "pageable memory, ids into a reused page-locked numpy "
                   "buffer") if not batch else
                  ("host documents in, each in its own pageable buffer -> "
                   "host uint32 ids, into a reused page-locked numpy buffer, "
                   "and row offsets out (tk_engine_encode_batch_docs, "
                   "transfers included)"),
        "latency_ms": pcts(host_lat),
        "mean_ms": round(host_ms, 4),
        "all_ms": [round(x, 3) for x in host_lat],
        "mchars_per_s": round(chars / (host_ms * 1e-3) / 1e6, 2),
        "tokens_per_s": round(n_tok / (host_ms * 1e-3), 1),
        "target_ms": TARGET_MS,
        "meets_target_p99": bool(pct(host_lat, 99) <= TARGET_MS),
    }
    if not batch:
        protocol["parts_us"] = {n: round(float(v), 1) for n, v in zip(
            ["bytes in (copy threads into the pinned staging)",
             "pipeline (one DMA in, the kernels, ids written into the "
             "page-locked buffer by k_compact)",
             "ids out (copy threads; none for a page-locked buffer)"],
            np.mean(np.asarray(m["host_parts"]), axis=0))}
        protocol["pageable_ids"] = {
            "window": "the same, ids into a reused pageable numpy buffer "
                      "(k_compact writes the engine's pinned staging, the "
                      "copy threads fill the buffer from it)",
            "latency_ms": pcts(m["plain_lat"]),
            "mean_ms": round(float(np.mean(m["plain_lat"])), 4),
            "parts_us": {n: round(float(v), 1) for n, v in zip(
                ["bytes in", "pipeline", "ids out"],
                np.mean(np.asarray(m["plain_parts"]), axis=0))},
        }
    rl = roofline(kname, launch_mean(m["kernel_us"]), b_alg,
                  measured_traffic(args.config, kname) if plain_traffic else None)
    rl["path_achieved"] = round(b_alg / (ms * 1e-3) / 1e9, 3)
    rl["chosen_by"] = ("the largest median own duration per request among "
                       f"{', '.join(names)} in the untimed stage pass over "
                       "the timed requests (every kernel timed); then timed "
                       "on its own dispatch in the timed region")
    line = {
        "metric": METRIC,
        "value": round(chars / (ms * 1e-3) / 1e6, 2),
        "unit": "Mchars/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic: seeded Zipf token-concat generator over the "
                "stand-in vocabulary of the family; every step a distinct "
                "seeded request",
        "config": {
            "workload": workload, "family": fam, "chars": int(chars),
            "bytes": int(n_bytes), "tokens": int(n_tok), "requests": K,
            "distinct_requests": True, "samples": [1, K + W],
            **({"rows_per_request": len(reqs[0])} if batch else {}),
        },
        "latency_ms": pcts(m["lat"]),
        "protocol": protocol,
        "host_to_host_ms": {"p50": protocol["latency_ms"]["p50"],
                            "p99": protocol["latency_ms"]["p99"]},
        "tokens_per_s": round(n_tok / (ms * 1e-3), 1),
        "stage_us": {n: round(float(v), 2) for n, v in zip(STAGE_NAMES, st[:, :4].mean(axis=0))},
        "kernels_us": kernel_summary(m["ku"]),
        "roofline": rl,
        "cpu_baseline": cpu,
        "cpu_lanes": lanes,
        "parity": {"checked": 0 if args.no_check else K, "mismatches": mism,
                   "against": "CPU oracle (C restatement), every timed request"
                              + (", every row" if batch else "")},
        "wall_s": round(m["wall"], 3),
    }
    tok.close()
    if (args.config == 2 and not (args.family or args.chat or args.seed
                                  or args.no_legs)):
        line["other_configs"] = {}
        for c in (3, 4, 5):
            lg = leg(c, max(1, args.leg_steps), 2, args.gen_workers)
            line["other_configs"][f"C{c}"] = lg
            mism += lg["parity"]["mismatches"]
    print(json.dumps(line), flush=True)
    return 0 if mism == 0 else 1


if __name__ == "__main__":
    sys.exit(main())
