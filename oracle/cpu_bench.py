"""CPU baseline leg of bench.py: the reference's own x86-64 code for every BASELINE.json config,
timed on this host's cores. TEST/BENCH INFRASTRUCTURE ONLY - it calls oracle/_ref/libkref.so
(the reference sources under /root/reference compiled by oracle/Makefile with the reference's
x86 flags), is imported only by bench.py's cpu_baseline leg, and is never the product path.

What runs (src/model/vllm_safetensors.c; x86 bodies - fp32 activations at M = 1, int16
activations for M > 1 and the default MoE track; a timing baseline, never a parity reference):
  config 1  dyn_matvec_q4_q8, K 2048 -> N 6144, M = 1 (q4_dense4_x86 row-group workers,
            :504-567, :1589-1595)
  config 2  the Qwen3-VL-2B decode-step linear set (fused QKV, O + residual, fused gate/up,
            down + residual) over 28 layers at M = 1 and 4 (the batched wrappers; from M = 2 on
            they take q4g_gemm_mat, :1583-1588, :1649, :1699-1702, :1754)
  config 3  Qwen3-8B gate (4096 -> 12288) and down (12288 -> 4096) at M = 1 (dense workers) and
            M = 2, 4, 8 (q4g_gemm_mat, :1130-1187)
  config 4  q4g_gemm_mat at M = 512 and 2048 (gate and down; M = 2048 takes the median of
            REPS_LONG calls, each a few hundred ms)
  config 5  st_moe_ffn_sparse_q4 (T = 1, :12921) and st_moe_ffn_sparse_q4_batch (T = 64,
            :14426) on the Qwen3-30B-A3B shape, in the default int16-activation track and in
            the int8 track (VLLM_ACTQ=1 VLLM_ACTQ16=0, :11431-11435). The track switch is read
            once per process, so the int8 track runs in a child process.
Method: the GPU run's seeded weights (kestrel-llm_amd/synth.py, same seeds and scales), cycled
over distinct copies whose total exceeds the host's last-level cache (the prefill GEMM, which
is compute-bound, uses two); two warm-up calls, then the median of >= 20 timed calls
(time.perf_counter, CLOCK_MONOTONIC). Thread counts: every physical core this process may run
on, and the reference's x86 default nc - 2 (src/core/vllm_tp.c:339), nc being the logical CPUs
available to the process (sysconf's count is reported beside it).
"""
import json
import os
import subprocess
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(ROOT, "kestrel-llm_amd"))

import oracle  # noqa: E402
import synth  # noqa: E402

REPS = 20
WARM = 2
REPS_LONG = 5      # config 4 at M = 2048
WARM_LONG = 1
ROTATE_MIN = 512 << 20


def host_info():
    """lscpu's sockets x cores x threads, the CPUs this process may use, and the physical cores
    among them (distinct (package, core) pairs)."""
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    cpus = sorted(os.sched_getaffinity(0))
    phys = set()
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f:
                pkg = f.read().strip()
            with open(base + "core_id") as f:
                core = f.read().strip()
            phys.add((pkg, core))
        except OSError:
            phys.add(("?", str(c)))
    llc = 0
    try:
        with open("/sys/devices/system/cpu/cpu0/cache/index3/size") as f:
            s = f.read().strip()
        llc = int(s[:-1]) * (1 << 10 if s.endswith("K") else 1 << 20) if s[-1] in "KM" else int(s)
    except (OSError, ValueError):
        pass
    return {
        "model": info.get("Model name", "?"),
        "lscpu": f"{info.get('Socket(s)', '?')} socket(s) x {info.get('Core(s) per socket', '?')} "
                 f"cores x {info.get('Thread(s) per core', '?')} threads",
        "cpus_available": len(cpus),
        "physical_cores_available": len(phys),
        "llc_bytes": llc,
    }


def median_us(fn, reps=REPS, warm=WARM):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)) * 1e6


def copies(arr, n):
    return [arr] + [arr.copy() for _ in range(n - 1)]


def n_rot(nbytes, llc):
    return max(2, -(-max(ROTATE_MIN, 4 * llc) // nbytes))


class Cycle:
    """Calls fn on the next weight copy each time."""

    def __init__(self, items, fn):
        self.items, self.fn, self.i = items, fn, 0

    def __call__(self):
        self.fn(self.items[self.i % len(self.items)])
        self.i += 1


P = lambda a: a.ctypes.data  # noqa: E731


def dense_configs(r, threads, llc, m_step):
    """Configs 1-4 at one thread count (the pool is re-initialised to `threads`)."""
    r.kref_init(threads)
    out = {}
    # config 1: single GEMV, the 2B FFN up-projection shape
    rows, cols = 6144, 2048
    w = synth.make_q4_weights(rows, cols, 11, **synth.SCALE_2B)
    ws = copies(w, n_rot(w.nbytes, llc))
    x = synth.make_activations(1, cols, 7)
    o = np.empty((1, rows), np.float32)
    us = median_us(Cycle(ws, lambda W: r.kref_matvec(P(o), P(W), P(x), rows, cols)))
    out["config1_gemv_m1"] = {"us": round(us, 1),
                              "GBs": round((w.nbytes + cols * 4 + rows * 4) / us / 1e3, 2)}
    del ws
    # config 2: the 2B decode-step linear set over 28 distinct layer copies
    cfg = synth.QWEN3VL_2B
    shapes = {n: (rr, cc) for n, rr, cc in synth.layer_shapes(cfg)}
    base = {n: synth.make_q4_weights(rr, cc, 1 + i, **synth.SCALE_2B)
            for i, (n, (rr, cc)) in enumerate(shapes.items())}
    layers = [base] + [{k: v.copy() for k, v in base.items()} for _ in range(cfg["layers"] - 1)]
    h, f = cfg["hidden"], cfg["ffn"]
    q, kv = shapes["q"][0], shapes["k"][0]
    for m in sorted({1, 4, m_step}):
        x = synth.make_activations(m, h, 7)
        attn = synth.make_activations(m, q, 8)
        act = synth.make_activations(m, f, 9)
        res = synth.make_activations(m, h, 10)
        b = {k: np.empty((m, n), np.float32) for k, n in
             dict(q=q, k=kv, v=kv, o=h, g=f, u=f, d=h).items()}

        def step():
            for L in layers:
                r.kref_qkv_batched(P(b["q"]), P(b["k"]), P(b["v"]), P(L["q"]), P(L["k"]),
                                   P(L["v"]), P(x), q, kv, h, m)
                r.kref_o_residual_batched(P(b["o"]), P(res), P(L["o"]), P(attn), h, q, m)
                r.kref_gate_up_batched(P(b["g"]), P(b["u"]), P(L["gate"]), P(L["up"]), P(x),
                                       f, h, m)
                r.kref_down_residual_batched(P(b["d"]), P(res), P(L["down"]), P(act), h, f, m)
        us = median_us(step)
        wb = sum(rr * cc * 18 // 32 for rr, cc in shapes.values())
        byts = cfg["layers"] * (wb + m * 4 * (h + q + h + f) + m * 4 * (q + 2 * kv + h + 2 * f + h)
                                + m * 4 * 2 * h)
        out[f"config2_step_m{m}"] = {"us": round(us, 1), "GBs": round(byts / us / 1e3, 2)}
    del layers, base
    # configs 3 and 4: Qwen3-8B gate and down
    cfg = synth.QWEN3_8B
    h, f = cfg["hidden"], cfg["ffn"]
    G = synth.make_q4_weights(f, h, 11, **synth.SCALE_8B)
    D = synth.make_q4_weights(h, f, 13, **synth.SCALE_8B)
    nr = n_rot(G.nbytes, llc)
    Gs, Ds = copies(G, nr), copies(D, nr)
    for m in (1, 2, 4, 8, 512, 2048):
        xg = synth.make_activations(m, h, 20 + m)
        xd = synth.make_activations(m, f, 30 + m)
        og, od = np.empty((m, f), np.float32), np.empty((m, h), np.float32)
        gs, ds = (Gs, Ds) if m <= 8 else (Gs[:2], Ds[:2])
        rw = dict(reps=REPS_LONG, warm=WARM_LONG) if m >= 2048 else {}
        if m == 1:
            tg = median_us(Cycle(gs, lambda W: r.kref_matvec(P(og), P(W), P(xg), f, h)))
            td = median_us(Cycle(ds, lambda W: r.kref_matvec(P(od), P(W), P(xd), h, f)))
        else:
            tg = median_us(Cycle(gs, lambda W: r.kref_gemm_mat(P(og), None, P(W), P(xg), f, h, m)),
                           **rw)
            td = median_us(Cycle(ds, lambda W: r.kref_gemm_mat(P(od), None, P(W), P(xd), h, f, m)),
                           **rw)
        if m <= 8:
            out[f"config3_m{m}"] = {
                "gate_us": round(tg, 1), "gate_GBs": round((G.nbytes + m * 4 * (h + f)) / tg / 1e3, 2),
                "down_us": round(td, 1), "down_GBs": round((D.nbytes + m * 4 * (h + f)) / td / 1e3, 2)}
        else:
            ops = 2.0 * m * f * h
            out[f"config4_m{m}"] = {"gate_us": round(tg, 1), "gate_GOPS": round(ops / tg / 1e3, 1),
                                    "down_us": round(td, 1), "down_GOPS": round(ops / td / 1e3, 1)}
    return out


def moe_track(r, threads_list, moe_file, llc):
    """Config 5 in the process's MoE track, at each thread count."""
    cfg = synth.QWEN3_30B_A3B_MOE
    d, ne, tk, ef = cfg["hidden"], cfg["experts"], cfg["top_k"], cfg["ef"]
    z = np.load(moe_file, mmap_mode="r")
    G, U, D = (np.ascontiguousarray(z[k]) for k in ("G", "U", "D"))
    router = (np.random.default_rng(62).standard_normal((ne, d), dtype=np.float32)
              * np.float32(0.02))
    per_copy = G.nbytes + U.nbytes + D.nbytes
    lay = [(G, U, D)] + [(G.copy(), U.copy(), D.copy()) for _ in range(n_rot(per_copy, llc) - 1)]
    res = {}
    for th in threads_list:
        r.kref_init(th)
        row = {}
        for T in (1, 64):
            X = synth.make_activations(T, d, 60)
            Y = np.empty((T, d), np.float32)
            us = median_us(Cycle(lay, lambda L: r.kref_moe_ffn(P(Y), P(X), T, P(router), P(L[0]),
                                                              P(L[1]), P(L[2]), ne, tk, d, ef)))
            row[f"T{T}_us"] = round(us, 1)
        res[str(th)] = row
    return res


def child_main(argv):
    """bench child: python oracle/cpu_bench.py --moe-track MOE_FILE LLC THREADS..."""
    moe_file, llc = argv[1], int(argv[2])
    threads = [int(t) for t in argv[3:]]
    with StdoutToStderr():
        r = oracle.ref(threads[0])
        res = moe_track(r, threads, moe_file, llc)
    print(json.dumps(res))


class StdoutToStderr:
    """The reference prints status lines with printf; while it runs, file descriptor 1 points at
    stderr so the bench's stdout carries only its JSON line."""

    def __enter__(self):
        sys.stdout.flush()
        self.saved = os.dup(1)
        os.dup2(2, 1)

    def __exit__(self, *exc):
        import ctypes
        ctypes.CDLL(None).fflush(None)
        os.dup2(self.saved, 1)
        os.close(self.saved)


def run(m_step=1):
    """The whole CPU baseline; returns the bench line's cpu_baseline object."""
    with StdoutToStderr():
        return _run(m_step)


def _run(m_step):
    if not oracle.ref_available():
        raise RuntimeError("oracle/_ref/libkref.so is not built (make -C oracle on a machine "
                           "with /root/reference); the CPU baseline times the reference's code")
    host = host_info()
    r = oracle.ref(1)
    nc_sys = int(r.kref_num_cpus())
    nc = min(nc_sys, host["cpus_available"])
    phys = host["physical_cores_available"]
    threads = [phys] + ([nc - 2] if nc > 2 and nc - 2 != phys else [])
    llc = host["llc_bytes"]
    t0 = time.perf_counter()
    dense = {str(th): dense_configs(r, th, llc, m_step) for th in threads}
    # MoE weights generated once, shared with the int8-track child through a file
    cfg = synth.QWEN3_30B_A3B_MOE
    G, U, D = synth.make_moe(cfg, 50)
    try:
        fd, moe_file = tempfile.mkstemp(suffix=".npz", dir="/dev/shm")
    except OSError:
        fd, moe_file = tempfile.mkstemp(suffix=".npz")
    os.close(fd)
    try:
        np.savez(moe_file, G=G, U=U, D=D)
        del G, U, D
        moe = {"int16_track": moe_track(r, threads, moe_file, llc)}
        env = dict(os.environ, VLLM_ACTQ="1", VLLM_ACTQ16="0")
        p = subprocess.run([sys.executable, os.path.abspath(__file__), "--moe-track", moe_file,
                            str(llc)] + [str(t) for t in threads],
                           capture_output=True, text=True, env=env, timeout=900)
        if p.returncode != 0:
            raise RuntimeError(f"int8-track child failed: {p.stderr[-2000:]}")
        moe["int8_track"] = json.loads(p.stdout.strip().splitlines()[-1])
    finally:
        os.unlink(moe_file)
    wall = time.perf_counter() - t0
    head = dense[str(phys)][f"config2_step_m{m_step}"]
    alt = ""
    if len(threads) > 1:
        h2 = dense[str(threads[1])][f"config2_step_m{m_step}"]
        alt = (f"; at the reference's own default of nc - 2 = {threads[1]} threads "
               f"(src/core/vllm_tp.c:339) {h2['GBs']} GB/s, {h2['us'] / 1e3:.2f} ms per step")
    return {
        "value": head["GBs"], "unit": "GB/s", "cores": phys, "kind": "reference",
        "sample": (f"config 2 (Qwen3-VL-2B decode-step linear set, 28 layers, M={m_step}): median "
                   f"of {REPS} steps of the reference's x86 wrappers; value is the run at every "
                   f"physical core ({phys} threads), {head['us'] / 1e3:.2f} ms per step{alt}; "
                   f"the other configs below, {wall:.0f} s in all"),
        "host": dict(host, nc_sysconf=nc_sys, nc=nc, threads=threads),
        "method": f"median of {REPS} calls after {WARM} warm-up calls; seeded weights as the GPU "
                  "run, cycled over copies beyond the LLC; reference x86 flags",
        "by_threads": dense,
        "moe_config5": moe,
        "moe_note": ("the int8 track's times sit on 4-ms steps: they measure the reference "
                     "thread pool's park/wake (src/core/vllm_tp.c), not its kernels; the int16 "
                     "track (the reference's x86 default) is the MoE figure to compare"),
    }


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "--moe-track":
        child_main(sys.argv[1:])
    else:
        print(json.dumps(run(int(sys.argv[1]) if len(sys.argv) > 1 else 1), indent=1))
