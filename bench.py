"""DF-J benchmark: screened density-fitted Coulomb forward + backward on one MI355X.

One step = E_J = 1/2 gamma^T (V + lam I)^-1 gamma over the screened pair list plus its full
reverse pass (J, every splat gradient and dC), with the refresh products (pair list, aux,
Cholesky factor, pair index) built beforehand and timed separately. Inputs are the seeded
synthetic systems of gs-dft_amd/workloads.py, resident in HBM before the timed region.

Prints one JSON line. ``value`` is three-centre integrals per second through the whole step
(N_aux x n_pairs integrals, each evaluated in the forward and again with derivatives in the
reverse pass); ``ms_per_step`` is the fwd+bwd wall time.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_FP64 = 78.6e12          # MI355X FP64 (vector and matrix) FLOP/s
PEAK_HBM = 8.0e12            # MI355X HBM3E bytes/s
# Algorithmic FP64 work per three-centre integral (P,a) at 20 nodes, transcendentals (rsqrt, exp)
# counted as one flop each: a per-integral prologue/epilogue plus a per-node part.
NODES = 20
FWD_PER_INTEGRAL, FWD_PER_NODE = 39, 17 + 2
BWD_PER_INTEGRAL, BWD_PER_NODE = 40, 35 + 2
FLOPS_FWD = FWD_PER_INTEGRAL + NODES * FWD_PER_NODE     # 419
FLOPS_BWD = BWD_PER_INTEGRAL + NODES * BWD_PER_NODE     # 780
METRIC = "DF-J fwd+bwd wall ms; 3-centre integrals/s; % of MI355X FP64 peak"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo) and its logical CPU count."""
    name = "unknown"
    try:
        for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return f"{name} ({os.cpu_count()} logical CPUs visible)"


def counter_record(workload: str, kernel: str):
    """The FP64 VALU counter figures of ``kernel`` at ``workload`` from the rocprofv3 counter runs
    summarised in profiles/three_centre_fp64_counters.json (None when not recorded)."""
    f = ROOT / "profiles" / "three_centre_fp64_counters.json"
    if not f.exists():
        return None
    return json.loads(f.read_text()).get(workload, {}).get(kernel)


def _with_command(out: dict) -> dict:
    """The JSON line with the command line that produced it."""
    return {**out, "command": "python bench.py " + " ".join(sys.argv[1:])}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--system", type=int, default=None,
                    help="benchmark system 1..5 (default 5; 3 for --term exact / exchange)")
    ap.add_argument("--eps", type=float, default=None,
                    help="screening threshold (default: the configuration's, 1e-7); the C20H42 "
                         "configuration is also quoted at 1e-5 and 1e-9")
    ap.add_argument("--pad-from-eps", type=float, default=None,
                    help="DF-J term: size the frozen pad (ceil(2 n0 / G) G) from the pair count "
                         "at this threshold instead of --eps, as a trainer does with its first "
                         "list; with a smaller --eps the list then stands for one grown within "
                         "that pad")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="target CPU time of the oracle baseline sample (0 disables it)")
    ap.add_argument("--cpu-sample-frac", type=float, default=0.0,
                    help="DF-J term: sample this fraction of the pair list for the CPU baseline "
                         "instead of sizing the sample by --cpu-seconds")
    ap.add_argument("--term", choices=("dfj", "nuclear", "exact", "grid", "exchange", "screen"),
                    default="dfj",
                    help="dfj: the screened DF-J step (the headline); nuclear: the screened "
                         "nuclear attraction E_ext with every gradient on the same pair list; "
                         "exact: the exact screened Coulomb E_J with every gradient (O(n^2), "
                         "system 3 unless --system is given); grid: rho and grad rho on an "
                         "atom-centred grid with every gradient; exchange: the screened RI-K "
                         "E_K with every gradient (system 3 unless --system is given); "
                         "screen: the pair-list build, dense scan against spatial candidates "
                         "(system 6 = the 60000-splat globule2100 screening shape)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 2 GiB device-to-device once (scales the HBM byte counters "
                         "FETCH_SIZE / WRITE_SIZE of a profiler run) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        x = torch.ones(1 << 28, dtype=torch.float64, device="cuda")
        y = torch.empty_like(x)
        torch.cuda.synchronize()
        y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": x.numel() * 8}), flush=True)
        return 0
    if args.gpus != 1:
        print(f"bench.py: the DF-J path is measured on one GPU only; --gpus {args.gpus} is not "
              f"run (sharding over several GPUs is designed, not built)", file=sys.stderr)
        return 2

    if args.system is None:
        args.system = 3 if args.term in ("exact", "exchange") else 5
    if args.term == "nuclear":
        return run_nuclear(args)
    if args.term == "exact":
        return run_exact(args)
    if args.term == "grid":
        return run_grid(args)
    if args.term == "exchange":
        return run_exchange(args)
    if args.term == "screen":
        return run_screen(args)

    import numpy as np
    import torch
    import __graft_entry__ as ge

    g = ge.load_package()
    import importlib
    wl = importlib.import_module("gs_dft_amd.workloads")
    from gs_dft_amd import _lib

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    s = wl.make_system(args.system, **({} if args.eps is None else {"eps": args.eps}))
    log(f"system {args.system} {s.name}: M={s.M} N_aux={s.n_aux} k={s.k} eps={s.eps}")

    quat = torch.tensor(s.quat, device=dev)
    ls = torch.tensor(s.log_scale, device=dev)
    cen = torch.tensor(s.centers, device=dev)
    C0 = torch.tensor(s.C, device=dev)
    occ = torch.tensor(s.occ, device=dev)
    ks = g.SplatDFJ(coulomb=g.df(scales=s.scales, lam=s.lam),
                    screen=g.pairlist(s.eps, unique=s.unique, skip_pad=True))

    # ------------------------------------------------------------------ refresh (timed apart)
    _lib.profile_enable(True)
    basis0 = g.Splat(quat=quat, log_scale=ls, centers=cen)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n0 = g.count_significant(basis0, s.eps if args.pad_from_eps is None else args.pad_from_eps,
                             s.unique)
    pad_to = g.train_pad_to(ks.screen, n0)
    t_count = time.perf_counter() - t0
    t0 = time.perf_counter()
    state = g.refresh(ks, basis0, pad_to=pad_to)
    torch.cuda.synchronize()
    t_refresh = time.perf_counter() - t0
    n = state.pair_index.n_live
    N = s.n_aux
    screen_ms = _lib.profile_read(_lib.PROF_SCREEN, reset=True)[0]
    metric_ms = _lib.profile_read(_lib.PROF_METRIC, reset=True)[0]
    chol_ms = _lib.profile_read(_lib.PROF_CHOLESKY, reset=True)[0]
    log(f"refresh: n_pairs={n} pad={pad_to} total {t_refresh * 1e3:.1f} ms "
        f"(screening call {screen_ms:.1f} ms between its events, the first call's code loading "
        f"and count read-back included -- bench.py --term screen times the kernels; metric "
        f"{metric_ms:.1f} ms, cholesky {chol_ms:.1f} ms)")

    # ------------------------------------------------------------------ step
    def step():
        b = g.Splat(quat=quat.clone().requires_grad_(), log_scale=ls.clone().requires_grad_(),
                    centers=cen.clone().requires_grad_())
        C = C0.clone().requires_grad_()
        E = ks(g.SplatModel(basis=b, C=C, occupations=occ), state)
        E.backward()
        return E

    for w in range(args.warmup):
        log(f"warmup step {w + 1}/{args.warmup}")
        step()
    torch.cuda.synchronize()
    for kid in (_lib.PROF_GAMMA_FWD, _lib.PROF_GAMMA_BWD, _lib.PROF_SOLVE):
        _lib.profile_read(kid, reset=True)
        _lib.profile_read_work(kid, reset=True)
    t0 = time.perf_counter()
    for k in range(args.steps):
        E = step()
        log(f"timed step {k + 1}/{args.steps}")
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    fwd_ms, fwd_n = _lib.profile_read(_lib.PROF_GAMMA_FWD, reset=True)
    bwd_ms, bwd_n = _lib.profile_read(_lib.PROF_GAMMA_BWD, reset=True)
    solve_ms, _ = _lib.profile_read(_lib.PROF_SOLVE, reset=True)
    fwd_nodes = _lib.profile_read_work(_lib.PROF_GAMMA_FWD, reset=True) / max(fwd_n, 1)
    bwd_nodes = _lib.profile_read_work(_lib.PROF_GAMMA_BWD, reset=True) / max(bwd_n, 1)
    fwd_ms /= max(fwd_n, 1)
    bwd_ms /= max(bwd_n, 1)
    _lib.profile_enable(False)
    integrals = float(N) * float(n)
    fwd_tf = integrals * FLOPS_FWD / (fwd_ms * 1e-3)
    bwd_tf = integrals * FLOPS_BWD / (bwd_ms * 1e-3)
    # What the kernels executed: the node screen leaves out nodes whose terms are below e^-36.
    fwd_exec_tf = (integrals * FWD_PER_INTEGRAL + fwd_nodes * FWD_PER_NODE) / (fwd_ms * 1e-3)
    bwd_exec_tf = (integrals * BWD_PER_INTEGRAL + bwd_nodes * BWD_PER_NODE) / (bwd_ms * 1e-3)
    fwd_node_frac = fwd_nodes / (NODES * integrals)
    bwd_node_frac = bwd_nodes / (NODES * integrals)
    log(f"E_J={E.item():.12e} step {wall * 1e3:.1f} ms; three-centre fwd {fwd_ms:.1f} ms "
        f"({fwd_tf / 1e12:.2f} TFLOP/s per integral, {fwd_exec_tf / 1e12:.2f} executed, "
        f"{100 * fwd_node_frac:.1f}% of nodes), bwd {bwd_ms:.1f} ms ({bwd_tf / 1e12:.2f} / "
        f"{bwd_exec_tf / 1e12:.2f} TFLOP/s, {100 * bwd_node_frac:.1f}% of nodes), "
        f"solves {solve_ms / max(args.steps, 1):.2f} ms")
    if bwd_ms >= fwd_ms:
        dom = ("reverse", "k_gamma_bwd", bwd_ms, FLOPS_BWD, bwd_tf, bwd_exec_tf, bwd_node_frac,
               BWD_PER_INTEGRAL, BWD_PER_NODE)
    else:
        dom = ("forward", "k_gamma_fwd", fwd_ms, FLOPS_FWD, fwd_tf, fwd_exec_tf, fwd_node_frac,
               FWD_PER_INTEGRAL, FWD_PER_NODE)
    # HBM bytes of the dominant kernel from the copy-calibrated counter runs of this workload,
    # stored per step together with the kernel's launches per step (the reverse runs its aux
    # slabs in several launches when their moments do not fit one launch's budget).
    traffic, launches = None, 1
    tfile = ROOT / "profiles" / "three_centre_traffic.json"
    if tfile.exists():
        rec = json.loads(tfile.read_text()).get(s.name, {}).get(dom[1])
        if rec:
            launches = int(rec.get("launches_per_step", 1))
            traffic = (rec["fetch_bytes"] + rec["write_bytes"]) / launches

    # ------------------------------------------------------------------ CPU baseline (oracle)
    cpu = None
    if args.cpu_seconds > 0:
        from oracle import oracle as orc
        pi, pj, w = (t.detach().cpu().numpy() for t in state.pairs)
        pi, pj, w = pi[:n], pj[:n], w[:n]
        la = state.aux.log_alpha.cpu().numpy()
        ac = state.aux.centers.cpu().numpy()
        d = np.random.default_rng(0).normal(size=N)
        rng = np.random.default_rng(1)

        def run(m, chunk=None):
            # A seeded random sample of m list entries against all aux functions, timed in
            # chunks of at most `chunk` entries (one progress line per chunk).
            sel = np.sort(rng.choice(n, size=min(m, n), replace=False))
            chunk = len(sel) if chunk is None else max(1, chunk)
            total = 0.0
            for c0 in range(0, len(sel), chunk):
                sc = sel[c0:c0 + chunk]
                t = time.perf_counter()
                orc.gamma(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi[sc], pj[sc],
                          w[sc])
                orc.gamma_vjp(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi[sc], pj[sc],
                              w[sc], d)
                total += time.perf_counter() - t
                if chunk < len(sel):
                    log(f"cpu baseline: {min(c0 + chunk, len(sel))} of {len(sel)} sampled pairs, "
                        f"{total:.1f} s")
            return total, len(sel)

        probe = max(1, min(n, int(2e6 // N) + 1))
        t_probe, m_probe = run(probe)
        m = max(1, min(n, int(m_probe * args.cpu_seconds / max(t_probe, 1e-6))))
        if args.cpu_sample_frac > 0:
            m = max(1, min(n, int(round(args.cpu_sample_frac * n))))
        per_chunk = max(m_probe, int(m_probe * 20.0 / max(t_probe, 1e-6)))   # ~20 s per chunk
        t_cpu, m_cpu = run(m, per_chunk) if m > m_probe else (t_probe, m_probe)
        per_pair = t_cpu / m_cpu
        cpu_step_ms = per_pair * n * 1e3
        cpu = {"value": cpu_step_ms, "unit": "ms per fwd+bwd step (three-centre gamma + reverse, "
               "extrapolated linearly in pairs)", "cores": orc.num_threads(), "kind": "port",
               "sample": f"{m_cpu} of {n} pairs ({100.0 * m_cpu / n:.3g}%) x all {N} aux "
                         f"functions, {t_cpu:.1f} s on {orc.num_threads()} threads (C oracle, "
                         f"OpenMP); metric, Cholesky and solves excluded",
               "sample_frac": m_cpu / n, "cpu_model": cpu_model(),
               "integrals_per_s": integrals / (cpu_step_ms * 1e-3)}
        log(f"cpu baseline: {cpu_step_ms / 1e3:.1f} s per step extrapolated from {m_cpu} pairs")

    out = {
        "metric": METRIC,
        "value": integrals / wall,
        "unit": "three-centre integrals/s (fwd+bwd step)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": f"{s.name}: screened DF-J fwd+bwd, M={s.M} splats, "
                               f"N_aux={N}, k={s.k}, eps={s.eps}, unique pairs",
                   "system": args.system, "M": s.M, "N_aux": N, "k": s.k, "n_pairs": n,
                   "pad_to": pad_to, "eps": s.eps, "parallelism": "single GPU",
                   **({} if args.pad_from_eps is None else
                      {"pad_from_eps": args.pad_from_eps, "n0_at_pad_eps": n0,
                       "n_pairs_over_n0": n / n0})},
        "roofline": {"bound": "valu", "kernel": f"three-centre {dom[0]} ({dom[1]})",
                     "achieved": dom[5] / 1e12, "peak": PEAK_FP64 / 1e12, "unit": "TFLOP/s",
                     "frac": dom[5] / PEAK_FP64, "frac_basis": "evaluated nodes",
                     "traffic": traffic, "launches_per_step": launches,
                     "flops_per_integral": dom[7], "flops_per_evaluated_node": dom[8],
                     "integrals_per_launch": integrals / launches,
                     "evaluated_nodes_per_launch": dom[6] * NODES * integrals / launches,
                     "kernel_ms_per_launch": dom[2] / launches, "kernel_ms_per_step": dom[2],
                     "nodes_evaluated_frac": dom[6],
                     "algorithmic_achieved": dom[4] / 1e12,
                     "algorithmic_frac": dom[4] / PEAK_FP64,
                     "algorithmic_flops_per_integral": dom[3],
                     "fp64_counters": counter_record(s.name, dom[1]),
                     "note": "FP64 compute bound on the vector ALUs (VALU; MI355X FP64 vector "
                             "peak 78.6 TFLOP/s, no MFMA: the work is elementwise). achieved "
                             "counts the work the kernel has to do: flops_per_integral for "
                             "every (P, a) plus flops_per_evaluated_node for each node the "
                             "e^-36 screen keeps (the kernel's own node counter); "
                             "algorithmic_* credit all 20 nodes of every integral, skipped ones "
                             "included, and so can pass 1; fp64_counters holds the hardware "
                             "FP64 VALU instruction rate of the same kernel at this workload "
                             "from the rocprofv3 counter runs in profiles/"},
        "kernels": {"three_centre_fwd_ms": fwd_ms, "three_centre_bwd_ms": bwd_ms,
                    "fwd_frac_fp64": fwd_exec_tf / PEAK_FP64,
                    "bwd_frac_fp64": bwd_exec_tf / PEAK_FP64,
                    "fwd_algorithmic_frac_fp64": fwd_tf / PEAK_FP64,
                    "bwd_algorithmic_frac_fp64": bwd_tf / PEAK_FP64,
                    "fwd_nodes_evaluated_frac": fwd_node_frac,
                    "bwd_nodes_evaluated_frac": bwd_node_frac,
                    "fwd_integrals_per_s": integrals / (fwd_ms * 1e-3),
                    "solves_ms": solve_ms / max(args.steps, 1),
                    "solves_hbm_gbs": 8.0 * N * N / (solve_ms / max(args.steps, 1) * 1e-3) / 1e9},
        "refresh_ms": {"total": t_refresh * 1e3, "count": t_count * 1e3, "screening_call": screen_ms,
                       "metric": metric_ms, "cholesky": chol_ms},
        "ms_per_step_with_refresh": wall * 1e3 + t_refresh * 1e3,
        "cpu_baseline": cpu,
        "E_J": E.item(),
    }
    print(json.dumps(_with_command(out)), flush=True)
    return 0


# Nuclear attraction, per (nucleus, pair) integral at 20 nodes: one pass of the three-centre
# reverse kernel over point-charge records (the same per-integral figure) that also forms the
# nucleus' force from its node sums: A^2 d (15), the three coefficients (3) and the scaled vector
# (18), 36 flops per integral; the cross-lane sums are per wave, not per integral.
FLOPS_NUC_PAIR = FLOPS_BWD + 36                                        # 816


def run_nuclear(args) -> int:
    """E_ext = sum_a w_a P_a V_a over the screened pair list with all gradients (splat leaves, C,
    nuclear coordinates): one step = one library pass for the value and the moments, plus the
    per-splat and per-nucleus reductions."""
    import numpy as np
    import torch
    import __graft_entry__ as ge

    g = ge.load_package()
    import importlib
    wl = importlib.import_module("gs_dft_amd.workloads")
    from gs_dft_amd import _lib

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    s = wl.make_system(args.system, **({} if args.eps is None else {"eps": args.eps}))
    log(f"system {args.system} {s.name}: M={s.M} atoms={len(s.charges)} k={s.k} eps={s.eps}")
    mk = lambda a: torch.tensor(a, device=dev, dtype=torch.float64)
    quat, ls, cen, C0, R0 = mk(s.quat), mk(s.log_scale), mk(s.centers), mk(s.C), mk(s.atoms)
    occ, Z = mk(s.occ), mk(s.charges)
    basis0 = g.Splat(quat=quat, log_scale=ls, centers=cen)
    pi, pj, w = g.neighbor_pairs(basis0, s.eps, unique=True)
    n, A = int(pi.shape[0]), int(Z.shape[0])
    integrals = float(n) * A
    log(f"pairs n={n}, nuclei {A}: {integrals:.4e} (nucleus, pair) integrals per pass")

    def step():
        b = g.Splat(quat=quat.clone().requires_grad_(), log_scale=ls.clone().requires_grad_(),
                    centers=cen.clone().requires_grad_())
        C = C0.clone().requires_grad_()
        R = R0.clone().requires_grad_()
        E = g.screened_external_energy(b, C, occ, pi, pj, R, Z, valid=w)
        E.backward()
        return E

    _lib.profile_enable(True)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    for kid in (_lib.PROF_NUC_PAIRS, _lib.PROF_NUC_ATOMS):
        _lib.profile_read(kid, reset=True)
        _lib.profile_read_work(kid, reset=True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        E = step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    pair_ms, pair_k = _lib.profile_read(_lib.PROF_NUC_PAIRS, reset=True)
    atom_ms, atom_k = _lib.profile_read(_lib.PROF_NUC_ATOMS, reset=True)
    pair_nodes = _lib.profile_read_work(_lib.PROF_NUC_PAIRS, reset=True) / max(pair_k, 1)
    _lib.profile_read_work(_lib.PROF_NUC_ATOMS, reset=True)
    _lib.profile_enable(False)
    pair_ms /= max(pair_k, 1)
    atom_ms /= max(atom_k, 1)
    pair_tf = integrals * FLOPS_NUC_PAIR / (pair_ms * 1e-3)
    nuc_per_integral = FLOPS_NUC_PAIR - NODES * BWD_PER_NODE
    pair_exec_tf = (integrals * nuc_per_integral + pair_nodes * BWD_PER_NODE) / (pair_ms * 1e-3)
    log(f"E_ext={E.item():.12e} step {wall * 1e3:.2f} ms; pair pass with nuclear forces "
        f"{pair_ms:.2f} ms ({pair_exec_tf / 1e12:.2f} TFLOP/s on the evaluated nodes, "
        f"{pair_tf / 1e12:.2f} algorithmic, {pair_nodes / (NODES * integrals):.3f} of nodes), "
        f"force sums over pair blocks {atom_ms:.2f} ms")
    dom = ("pair pass with nuclear forces (k_gamma_bwd<false, true> over point-charge records)",
           pair_ms, FLOPS_NUC_PAIR, pair_tf, pair_exec_tf, nuc_per_integral)

    cpu = None
    if args.cpu_seconds > 0:
        from oracle import oracle as orc
        pin, pjn, wn = (t.cpu().numpy() for t in (pi, pj, w))
        rng = np.random.default_rng(1)

        def run(m):
            sel = np.sort(rng.choice(n, size=min(m, n), replace=False))
            t = time.perf_counter()
            orc.external_energy(s.quat, s.log_scale, s.centers, s.C, s.occ, pin[sel], pjn[sel],
                                wn[sel], s.atoms, s.charges)
            return time.perf_counter() - t, len(sel)

        t_probe, m_probe = run(max(1, min(n, 2000)))
        m = max(1, min(n, int(m_probe * args.cpu_seconds / max(t_probe, 1e-6))))
        t_cpu, m_cpu = run(m) if m > m_probe else (t_probe, m_probe)
        cpu_ms = t_cpu / m_cpu * n * 1e3
        cpu = {"value": cpu_ms, "unit": "ms per energy evaluation (extrapolated linearly in "
               "pairs)", "cores": orc.num_threads(), "kind": "port", "cpu_model": cpu_model(),
               "sample": f"{m_cpu} of {n} pairs x all {A} nuclei, {t_cpu:.1f} s on "
                         f"{orc.num_threads()} threads (C oracle, OpenMP); energy only: the "
                         f"oracle has no hand-written reverse pass for this term",
               "integrals_per_s": integrals / (cpu_ms * 1e-3)}
        log(f"cpu baseline: {cpu_ms / 1e3:.2f} s per energy extrapolated from {m_cpu} pairs")

    out = {
        "metric": "screened V_ne energy+gradients wall ms; (nucleus, pair) integrals/s",
        "value": integrals / wall,
        "unit": "(nucleus, pair) integrals/s (energy + all gradients)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": f"{s.name}: screened nuclear attraction, M={s.M} splats, "
                               f"{A} nuclei, k={s.k}, eps={s.eps}, unique pairs",
                   "system": args.system, "M": s.M, "n_atoms": A, "k": s.k, "n_pairs": n,
                   "eps": s.eps, "parallelism": "single GPU"},
        "roofline": {"bound": "valu", "kernel": dom[0], "achieved": dom[4] / 1e12,
                     "peak": PEAK_FP64 / 1e12, "unit": "TFLOP/s", "frac": dom[4] / PEAK_FP64,
                     "frac_basis": "evaluated nodes",
                     "traffic": None, "flops_per_integral": dom[5],
                     "flops_per_evaluated_node": BWD_PER_NODE,
                     "integrals_per_launch": integrals, "kernel_ms": dom[1],
                     "algorithmic_achieved": dom[3] / 1e12, "algorithmic_frac": dom[3] / PEAK_FP64,
                     "algorithmic_flops_per_integral": dom[2],
                     "note": "FP64 vector (VALU) bound; achieved counts flops_per_integral for "
                             "every (nucleus, pair) plus flops_per_evaluated_node for each node "
                             "the e^-36 screen keeps; algorithmic_* credit all 20 nodes of every "
                             "integral, skipped ones included"},
        "kernels": {"pair_pass_ms": pair_ms, "force_sums_ms": atom_ms,
                    "pair_nodes_evaluated_frac": pair_nodes / (NODES * integrals)},
        "cpu_baseline": cpu,
        "E_ext": E.item(),
    }
    print(json.dumps(_with_command(out)), flush=True)
    return 0


# Exact pair-pair Coulomb, per (a, b) integral at 20 nodes: a prologue of T = A_a^-1 + A_b^-1,
# d, adj T, the invariants J1..J3 and p0..p2 (~100 flops), then per node the three-centre node
# (17 + 2); the reverse adds the node moments (16 + 2 per node) and the chain to dF/dT, dF/dd
# (~120 flops).
ERI_FWD_PER_INTEGRAL, ERI_FWD_PER_NODE = 100, 19
ERI_BWD_PER_INTEGRAL, ERI_BWD_PER_NODE = 220, 37
FLOPS_ERI_FWD = ERI_FWD_PER_INTEGRAL + NODES * ERI_FWD_PER_NODE     # 480
FLOPS_ERI_BWD = ERI_BWD_PER_INTEGRAL + NODES * ERI_BWD_PER_NODE     # 960


def run_exact(args) -> int:
    """Exact E_J = 1/2 sum_{a,b} (a|b) Pw_a Pw_b over the screened pair list: one step = the energy
    with every gradient (one reverse pass over the n(n+1)/2 unordered pair-pairs plus the per-splat
    reductions); the energy-only evaluation is timed beside it. `value` counts the n^2 ordered
    pair-pair integrals the energy is defined over."""
    import numpy as np
    import torch
    import __graft_entry__ as ge

    g = ge.load_package()
    import importlib
    wl = importlib.import_module("gs_dft_amd.workloads")
    from gs_dft_amd import _lib

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    s = wl.make_system(args.system, **({} if args.eps is None else {"eps": args.eps}))
    log(f"system {args.system} {s.name}: M={s.M} k={s.k} eps={s.eps}")
    mk = lambda a: torch.tensor(a, device=dev, dtype=torch.float64)
    quat, ls, cen, C0, occ = mk(s.quat), mk(s.log_scale), mk(s.centers), mk(s.C), mk(s.occ)
    basis0 = g.Splat(quat=quat, log_scale=ls, centers=cen)
    pi, pj, w = g.neighbor_pairs(basis0, s.eps, unique=True)
    index = g.build_pair_index(s.M, pi, pj, w)
    n = int(pi.shape[0])
    integrals = float(n) * n
    sym_integrals = float(n) * (n + 1) / 2       # the energy-only pass evaluates (a|b) once
    log(f"pairs n={n}: {integrals:.4e} pair-pair integrals per pass")

    def step():
        b = g.Splat(quat=quat.clone().requires_grad_(), log_scale=ls.clone().requires_grad_(),
                    centers=cen.clone().requires_grad_())
        C = C0.clone().requires_grad_()
        E = g.screened_coulomb_energy(b, C, occ, pi, pj, valid=w, index=index)
        E.backward()
        return E

    _lib.profile_enable(True)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    for kid in (_lib.PROF_ERI_FWD, _lib.PROF_ERI_BWD):
        _lib.profile_read(kid, reset=True)
        _lib.profile_read_work(kid, reset=True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        E = step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    with torch.no_grad():
        t1 = time.perf_counter()
        E0 = g.screened_coulomb_energy(basis0, C0, occ, pi, pj, valid=w, index=index)
        torch.cuda.synchronize()
        wall_e = time.perf_counter() - t1
    bwd_ms, bwd_k = _lib.profile_read(_lib.PROF_ERI_BWD, reset=True)
    fwd_ms, fwd_k = _lib.profile_read(_lib.PROF_ERI_FWD, reset=True)
    bwd_nodes = _lib.profile_read_work(_lib.PROF_ERI_BWD, reset=True) / max(bwd_k, 1)
    fwd_nodes = _lib.profile_read_work(_lib.PROF_ERI_FWD, reset=True) / max(fwd_k, 1)
    _lib.profile_enable(False)
    bwd_ms /= max(bwd_k, 1)
    fwd_ms /= max(fwd_k, 1)
    bwd_tf = sym_integrals * FLOPS_ERI_BWD / (bwd_ms * 1e-3)
    fwd_tf = sym_integrals * FLOPS_ERI_FWD / (fwd_ms * 1e-3)
    bwd_exec_tf = (sym_integrals * ERI_BWD_PER_INTEGRAL + bwd_nodes * ERI_BWD_PER_NODE) / (
        bwd_ms * 1e-3)
    fwd_exec_tf = (sym_integrals * ERI_FWD_PER_INTEGRAL + fwd_nodes * ERI_FWD_PER_NODE) / (
        fwd_ms * 1e-3)
    log(f"E_J={E.item():.12e} (energy only {E0.item():.12e}) step {wall * 1e3:.1f} ms, energy "
        f"only {wall_e * 1e3:.1f} ms; reverse kernel {bwd_ms:.1f} ms ({bwd_tf / 1e12:.2f} "
        f"TFLOP/s, {bwd_nodes / (NODES * sym_integrals):.3f} of nodes), forward kernel "
        f"{fwd_ms:.1f} ms ({fwd_tf / 1e12:.2f} TFLOP/s over the n(n+1)/2 unordered pair-pairs, "
        f"{fwd_nodes / (NODES * sym_integrals):.3f})")

    cpu = None
    if args.cpu_seconds > 0:
        from oracle import oracle as orc
        pin, pjn, wn = (t.cpu().numpy() for t in (pi, pj, w))
        rng = np.random.default_rng(1)

        def run(m):
            sel = np.sort(rng.choice(n, size=min(m, n), replace=False))
            t = time.perf_counter()
            orc.eri_block(s.quat, s.log_scale, s.centers, pin[sel], pjn[sel], pin, pjn)
            return time.perf_counter() - t, len(sel)

        t_probe, m_probe = run(max(1, min(n, int(2e6 // n) + 1)))
        m = max(1, min(n, int(m_probe * args.cpu_seconds / max(t_probe, 1e-6))))
        t_cpu, m_cpu = run(m) if m > m_probe else (t_probe, m_probe)
        cpu_ms = t_cpu / m_cpu * n * 1e3
        cpu = {"value": cpu_ms, "unit": "ms per energy evaluation (all (a|b), extrapolated "
               "linearly in bra pairs)", "cores": orc.num_threads(), "kind": "port",
               "cpu_model": cpu_model(),
               "sample": f"{m_cpu} of {n} bra pairs x all {n} ket pairs, {t_cpu:.1f} s on "
                         f"{orc.num_threads()} threads (C oracle, OpenMP, the reference's Schur "
                         f"node form); energy only",
               "integrals_per_s": integrals / (cpu_ms * 1e-3)}
        log(f"cpu baseline: {cpu_ms / 1e3:.1f} s per energy extrapolated from {m_cpu} bra pairs")

    out = {
        "metric": "exact screened E_J fwd+bwd wall ms; pair-pair integrals/s",
        "value": integrals / wall,
        "unit": "pair-pair integrals/s (energy + all gradients)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": f"{s.name}: exact screened Coulomb, M={s.M} splats, k={s.k}, "
                               f"eps={s.eps}, unique pairs",
                   "system": args.system, "M": s.M, "k": s.k, "n_pairs": n, "eps": s.eps,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "valu", "kernel": "exact pair-pair reverse (k_eri_bwd_sym, all bands)",
                     "achieved": bwd_exec_tf / 1e12, "peak": PEAK_FP64 / 1e12, "unit": "TFLOP/s",
                     "frac": bwd_exec_tf / PEAK_FP64, "frac_basis": "evaluated nodes",
                     "traffic": None, "flops_per_integral": ERI_BWD_PER_INTEGRAL,
                     "flops_per_evaluated_node": ERI_BWD_PER_NODE,
                     "integrals_per_launch": sym_integrals, "kernel_ms": bwd_ms,
                     "algorithmic_achieved": bwd_tf / 1e12, "algorithmic_frac": bwd_tf / PEAK_FP64,
                     "algorithmic_flops_per_integral": FLOPS_ERI_BWD,
                     "note": "FP64 vector (VALU) bound, over the n(n+1)/2 unordered pair-pairs "
                             "each pass evaluates ((a|b) = (b|a)); achieved counts "
                             "flops_per_integral per pair-pair plus flops_per_evaluated_node "
                             "for each node the e^-36 screen keeps; algorithmic_* credit all 20 "
                             "nodes; kernel_ms spans every band launch and its reductions"},
        "kernels": {"reverse_ms": bwd_ms, "forward_ms": fwd_ms,
                    "energy_only_ms": wall_e * 1e3,
                    "forward_frac_fp64": fwd_exec_tf / PEAK_FP64,
                    "forward_algorithmic_frac_fp64": fwd_tf / PEAK_FP64,
                    "forward_pair_pairs": sym_integrals,
                    "reverse_nodes_evaluated_frac": bwd_nodes / (NODES * sym_integrals),
                    "forward_nodes_evaluated_frac": fwd_nodes / (NODES * sym_integrals)},
        "cpu_baseline": cpu,
        "E_J": E.item(),
    }
    print(json.dumps(_with_command(out)), flush=True)
    return 0


def run_exchange(args) -> int:
    """Screened RI-K E_K = -||L^-1 D||^2 with every gradient (splat leaves and C) on the ordered
    pair list and the frozen product aux: one step = per aux chunk the three-centre block, the
    pair-sparse Y = T_P C and the FP64 GEMM D_P = C^T Y_P, one triangular solve over the
    k(k+1)/2 packed columns, then the reverse (second solve, per chunk dC and Ybar GEMMs, the
    sampled Tbar and the three-centre reverse). The refresh products are built beforehand."""
    import numpy as np
    import torch
    import __graft_entry__ as ge

    g = ge.load_package()
    import importlib
    wl = importlib.import_module("gs_dft_amd.workloads")
    from gs_dft_amd import _lib

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    s = wl.make_system(args.system, **({} if args.eps is None else {"eps": args.eps}))
    mk = lambda a: torch.tensor(a, device=dev, dtype=torch.float64)
    quat, ls, cen, C0 = mk(s.quat), mk(s.log_scale), mk(s.centers), mk(s.C)
    basis0 = g.Splat(quat=quat, log_scale=ls, centers=cen)
    lam = 1e-8
    pi, pj, w = g.neighbor_pairs(basis0, s.eps, unique=False)
    index = g.build_pair_index(s.M, pi, pj, w)
    aux = g.init_product_aux(basis0, scales=s.scales)
    L = g.aux_cholesky(aux, lam)
    torch.cuda.synchronize()
    M, k, N, n = s.M, s.k, aux.n_basis, index.n_live
    K2 = k * (k + 1) // 2
    log(f"system {args.system} {s.name}: M={M} k={k} N_aux={N} ordered pairs n={n}")
    integrals = float(N) * n
    gemm_fwd = 2.0 * N * M * k * k                  # D_P = C^T Y_P
    gemm_bwd = 2.0 * (2.0 * N * M * k * k)          # dC += 2 Y_P Dbar_P, Ybar_P = C Dbar_P
    trsm = float(N) * N * K2                        # one solve over K2 columns
    sparse = 2.0 * 2.0 * N * n * k                  # Y = T C and Tbar = Ybar . C (symmetric list)
    flops = (gemm_fwd + gemm_bwd + 2 * trsm + sparse + integrals * (FLOPS_FWD + FLOPS_BWD))

    def step():
        b = g.Splat(quat=quat.clone().requires_grad_(), log_scale=ls.clone().requires_grad_(),
                    centers=cen.clone().requires_grad_())
        C = C0.clone().requires_grad_()
        E = g.df_exchange_energy_screened(b, C, aux, pi, pj, lam=lam, valid=w, cholV=L,
                                          index=index)
        E.backward()
        return E

    ids = (_lib.PROF_EXCH_BLOCK, _lib.PROF_EXCH_BWD, _lib.PROF_EXCH_TRSM, _lib.PROF_EXCH_GEMM,
           _lib.PROF_EXCH_SPARSE)
    _lib.profile_enable(True)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    for kid in ids:
        _lib.profile_read(kid, reset=True)
        _lib.profile_read_work(kid, reset=True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        E = step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    prof = {kid: _lib.profile_read(kid, reset=True) for kid in ids}
    bwd_nodes = _lib.profile_read_work(_lib.PROF_EXCH_BWD, reset=True) / args.steps
    blk_nodes = _lib.profile_read_work(_lib.PROF_EXCH_BLOCK, reset=True) / args.steps
    _lib.profile_enable(False)
    # the three-centre passes run once per unordered splat pair (the list is symmetric)
    groups = int(((pi <= pj) & (w != 0)).sum().item())
    blk_exec = float(groups) * N * FWD_PER_INTEGRAL + blk_nodes * FWD_PER_NODE
    rev_exec = float(groups) * N * BWD_PER_INTEGRAL + bwd_nodes * BWD_PER_NODE
    per_step = {kid: prof[kid][0] / args.steps for kid in ids}
    blk_ms, rev_ms = per_step[_lib.PROF_EXCH_BLOCK], per_step[_lib.PROF_EXCH_BWD]
    trsm_ms, gemm_ms = per_step[_lib.PROF_EXCH_TRSM], per_step[_lib.PROF_EXCH_GEMM]
    sparse_ms = per_step[_lib.PROF_EXCH_SPARSE]
    trsm_tf = 2 * trsm / (trsm_ms * 1e-3)
    gemm_tf = (gemm_fwd + gemm_bwd) / (gemm_ms * 1e-3)
    with torch.no_grad():
        t1 = time.perf_counter()
        E0 = g.df_exchange_energy_screened(basis0, C0, aux, pi, pj, lam=lam, valid=w, cholV=L,
                                           index=index)
        torch.cuda.synchronize()
        wall_e = time.perf_counter() - t1
    log(f"E_K={E.item():.12e} (energy only {E0.item():.12e}); step {wall * 1e3:.1f} ms, energy "
        f"only {wall_e * 1e3:.1f} ms; per step: trsm {trsm_ms:.1f} ms ({trsm_tf / 1e12:.1f} "
        f"TFLOP/s), GEMMs {gemm_ms:.1f} ms ({gemm_tf / 1e12:.1f} TFLOP/s), three-centre block "
        f"{blk_ms:.1f} ms, three-centre reverse {rev_ms:.1f} ms, pair-sparse products "
        f"{sparse_ms:.1f} ms")
    # the dominant kernel family of the step and its algorithmic flops per step (work that a
    # recompute repeats is not counted again)
    # (name, ms per step, work the kernels do per step, algorithmic work per step, bound): the
    # three-centre passes do one integral per (group, aux) and the nodes the screen keeps, the
    # algorithmic figure counts every ordered entry at all 20 nodes, as the reference evaluates
    fams = [("three-centre block (k_exch_block)", blk_ms, blk_exec, integrals * FLOPS_FWD,
             "valu"),
            ("three-centre reverse (k_gamma_bwd, per-(P,a) cotangent)", rev_ms, rev_exec,
             integrals * FLOPS_BWD, "valu"),
            ("pair-sparse products (k_exch_spmm, k_exch_sddmm; FP64 MFMA)", sparse_ms, sparse,
             sparse, "mfma"),
            ("FP64 GEMMs (k_gemm_tn_sub, FP64 MFMA)", gemm_ms, gemm_fwd + gemm_bwd, gemm_fwd + gemm_bwd,
             "mfma"),
            ("triangular solves (blocked, k_panel_subst + FP64 MFMA products)", trsm_ms, 2 * trsm, 2 * trsm, "mfma")]
    dom = max(fams, key=lambda f: f[1])
    dom_tf = dom[2] / (dom[1] * 1e-3)
    dom_alg_tf = dom[3] / (dom[1] * 1e-3)
    # HBM bytes per launch (one aux chunk) of the dominant kernel, from the counter runs
    traffic, counters = None, None
    tkey = {"three-centre reverse": "k_gamma_bwd_lane_u",
            "three-centre block": "k_exch_block_pairs"}.get(dom[0].split(" (")[0])
    tfile = ROOT / "profiles" / "exchange_traffic.json"
    if tkey and tfile.exists():
        rec = json.loads(tfile.read_text()).get(s.name, {}).get(tkey)
        if rec:
            traffic = rec["fetch_bytes"] + rec["write_bytes"]
            counters = rec.get("fp64_counters")      # executed FP64 flops on hardware counters

    cpu = None
    if args.cpu_seconds > 0:
        from oracle import oracle as orc
        pin, pjn = pi.cpu().numpy(), pj.cpu().numpy()
        la, ac = aux.log_alpha.cpu().numpy(), aux.centers.cpu().numpy()
        rng = np.random.default_rng(1)

        def per_pair(m):           # the reference's D accumulation over m pairs (ri.py:524-531)
            sel = np.sort(rng.choice(n, size=min(m, n), replace=False))
            t = time.perf_counter()
            B = orc.three_center_block(s.quat, s.log_scale, s.centers, la, ac, pin[sel], pjn[sel])
            np.einsum("Ap,po,pq->Aoq", B, s.C[pin[sel]], s.C[pjn[sel]], optimize=True)
            return time.perf_counter() - t, len(sel)

        m_probe, t_probe = 4, 0.0
        while True:                 # grow the probe until it is long enough to scale from
            t_probe, m_probe = per_pair(m_probe)
            if t_probe > 0.5 or m_probe >= n:
                break
            m_probe *= 4
        m = max(m_probe, min(n, int(m_probe * 0.5 * args.cpu_seconds / max(t_probe, 1e-6))))
        t_pairs, m_pairs = per_pair(m) if m > m_probe else (t_probe, m_probe)
        Dr = rng.normal(size=(N, k, k))
        t = time.perf_counter()
        Mm = np.einsum("Aoq,Boq->AB", Dr, Dr, optimize=True)       # ri.py:532
        Vs = orc.aux_metric(la, ac, lam)
        np.trace(np.linalg.solve(Vs, Mm))                           # ri.py:544
        t_fixed = time.perf_counter() - t
        cpu_ms = (t_pairs / m_pairs * n + t_fixed) * 1e3
        cpu = {"value": cpu_ms, "unit": "ms per energy evaluation (pair part extrapolated "
               "linearly in pairs, plus the measured M build and solve)",
               "cores": orc.num_threads(), "kind": "port", "cpu_model": cpu_model(),
               "sample": f"{m_pairs} of {n} pairs x all {N} aux ({t_pairs:.1f} s) + M = D D^T "
                         f"and the dense solve at full size ({t_fixed:.1f} s) on "
                         f"{orc.num_threads()} threads (C oracle three-centre block, numpy "
                         f"einsum contractions as gs_dft/coulomb/ri.py:497-544); energy only"}
        log(f"cpu baseline: {cpu_ms / 1e3:.1f} s per energy ({m_pairs} pairs sampled)")

    out = {
        "metric": "screened RI-K fwd+bwd wall ms; algorithmic FP64 FLOP/s",
        "value": flops / wall,
        "unit": "algorithmic FP64 FLOP/s (energy + all gradients)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": f"{s.name}: screened RI-K exchange, M={M} splats, k={k}, "
                               f"N_aux={N}, eps={s.eps}, ordered pairs",
                   "system": args.system, "M": M, "k": k, "N_aux": N, "n_pairs": n,
                   "eps": s.eps, "parallelism": "single GPU"},
        "roofline": {"bound": dom[4], "kernel": dom[0], "achieved": dom_tf / 1e12,
                     "peak": PEAK_FP64 / 1e12, "unit": "TFLOP/s", "frac": dom_tf / PEAK_FP64,
                     "traffic": traffic, "flops_per_step": dom[2], "kernel_ms_per_step": dom[1],
                     "frac_basis": "evaluated nodes, one integral per unordered splat pair",
                     "algorithmic_achieved": dom_alg_tf / 1e12,
                     "algorithmic_frac": dom_alg_tf / PEAK_FP64,
                     "algorithmic_flops_per_step": dom[3], "pair_groups": groups,
                     "fp64_counters": counters,
                     "note": "per step, summed over the chunk launches; FP64 peak 78.6 (vector "
                             "and matrix). Three-centre passes: achieved counts, per unordered "
                             "splat pair (pair_groups) and aux function, the per-integral "
                             "prologue (39 block, 40 reverse) plus 19 (block) or 37 (reverse) "
                             "flops per node the e^-36 screen keeps; algorithmic_* count every "
                             "ordered entry at all 20 nodes (N n x 419 block, N n x 780 "
                             "reverse), as the reference evaluates them, and so can pass 1. "
                             "Other families: 4 N n k (Y = T C and Tbar), 6 N M k^2 (GEMMs), "
                             "2 N^2 K2 (solves). traffic is the dominant kernel's HBM bytes per "
                             "launch (one aux chunk) and fp64_counters its executed FP64 "
                             "flops, from the counter runs in profiles/"},
        "kernels": {"trsm_ms_per_step": trsm_ms, "trsm_tflops": trsm_tf / 1e12,
                    "gemm_ms_per_step": gemm_ms, "gemm_tflops": gemm_tf / 1e12,
                    "block_ms_per_step": blk_ms, "reverse_ms_per_step": rev_ms,
                    "sparse_ms_per_step": sparse_ms,
                    "reverse_nodes_evaluated_frac": bwd_nodes / (NODES * float(groups) * N),
                    "block_nodes_evaluated_frac": blk_nodes / (NODES * float(groups) * N),
                    "energy_only_ms": wall_e * 1e3},
        "cpu_baseline": cpu,
        "E_K": E.item(),
    }
    print(json.dumps(_with_command(out)), flush=True)
    return 0


def run_grid(args) -> int:
    """(rho, grad rho) on an atom-centred grid with every gradient (splat leaves and C): one step =
    the forward (basis values, psi = g C, phi = (psi occ) C^T) and the reverse (psi and grad psi,
    dC += [g; dg]^T [Pbar; Pbar_d], [gbar; dgbar] = [Pbar; Pbar_d] C^T, basis reverse)."""
    import numpy as np
    import torch
    import __graft_entry__ as ge

    g = ge.load_package()
    import importlib
    wl = importlib.import_module("gs_dft_amd.workloads")

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    s = wl.make_system(args.system, **({} if args.eps is None else {"eps": args.eps}))
    pts_np = wl.atom_grid(s.atoms, n_rad=16, n_ang=50, r_max=10.0, seed=args.system)
    G = int(pts_np.shape[0])
    M, k = s.M, s.k
    chunk = 8192
    log(f"system {args.system} {s.name}: M={M} k={k}, grid {G} points ({len(s.atoms)} atoms x 16 "
        f"radii x 50 directions), chunk {chunk}")
    mk = lambda a: torch.tensor(a, device=dev, dtype=torch.float64)
    quat, ls, cen, C0, occ, pts = (mk(a) for a in (s.quat, s.log_scale, s.centers, s.C, s.occ,
                                                   pts_np))
    v = mk(np.random.default_rng(0).uniform(0.5, 1.5, G))

    def step():
        b = g.Splat(quat=quat.clone().requires_grad_(), log_scale=ls.clone().requires_grad_(),
                    centers=cen.clone().requires_grad_())
        C = C0.clone().requires_grad_()
        rho, grad = g.chunked_density_and_grad(b, C, occ, pts, chunk=chunk)
        E = (v * rho).sum() + (grad * grad).sum()
        E.backward()
        return E

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        E = step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    with torch.no_grad():
        b0 = g.Splat(quat=quat, log_scale=ls, centers=cen)
        t1 = time.perf_counter()
        g.chunked_density_and_grad(b0, C0, occ, pts, chunk=chunk)
        torch.cuda.synchronize()
        wall_f = time.perf_counter() - t1
    # GEMM flops: forward psi = g C and phi = (psi occ) C^T; reverse [psi; dpsi] (4), dC (4),
    # [gbar; dgbar] (4), each 2 G M k
    gemm = 2.0 * G * M * k
    flops_step = gemm * (2 + 12)
    tf = flops_step / wall
    log(f"E={E.item():.12e} step {wall * 1e3:.1f} ms (forward only {wall_f * 1e3:.1f} ms): "
        f"{tf / 1e12:.2f} TFLOP/s of FP64 GEMM work through the step")
    cpu = None
    if args.cpu_seconds > 0:
        from oracle import torch_ref as tr
        torch.set_num_threads(max(1, os.cpu_count() or 1))
        rng = np.random.default_rng(1)
        args_t = [torch.as_tensor(a) for a in (s.quat, s.log_scale, s.centers, s.C, s.occ)]

        def run(m):
            sel = np.sort(rng.choice(G, size=min(m, G), replace=False))
            t = time.perf_counter()
            tr.chunked_density(*args_t, torch.as_tensor(pts_np[sel]), kind="gga", chunk=1024)
            return time.perf_counter() - t, len(sel)

        t_probe, m_probe = run(256)
        m = max(1, min(G, int(m_probe * args.cpu_seconds / max(t_probe, 1e-6))))
        t_cpu, m_cpu = run(m) if m > m_probe else (t_probe, m_probe)
        cpu_ms = t_cpu / m_cpu * G * 1e3
        cpu = {"value": cpu_ms, "unit": "ms per forward (rho, grad rho) evaluation, extrapolated "
               "linearly in grid points", "cores": torch.get_num_threads(), "kind": "port",
               "cpu_model": cpu_model(),
               "sample": f"{m_cpu} of {G} points, {t_cpu:.1f} s (torch float64 restatement of "
                         f"the reference on the host, {torch.get_num_threads()} threads); "
                         f"forward only"}
        log(f"cpu baseline: {cpu_ms / 1e3:.1f} s per forward extrapolated from {m_cpu} points")
    out = {
        "metric": "grid density (rho, grad rho) fwd+bwd wall ms; FP64 GEMM TFLOP/s",
        "value": tf / 1e12,
        "unit": "TFLOP/s (FP64 GEMM work of the step)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": f"{s.name}: rho and grad rho with all gradients, M={M} splats, "
                               f"k={k}, {G} grid points", "system": args.system, "M": M, "k": k,
                   "grid_points": G, "chunk": chunk, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "FP64 GEMMs of the step (the library's own FP64 MFMA product, k_gemm_tn_sub)",
                     "achieved": tf / 1e12, "peak": PEAK_FP64 / 1e12, "unit": "TFLOP/s",
                     "frac": tf / PEAK_FP64, "traffic": None,
                     "note": "whole-step rate: the basis kernels and reductions are counted as "
                             "time, not flops"},
        "kernels": {"forward_only_ms": wall_f * 1e3},
        "cpu_baseline": cpu,
    }
    print(json.dumps(_with_command(out)), flush=True)
    return 0


def run_screen(args) -> int:
    """The pair-list build at one system: count + build, by the dense tile scan over every
    candidate and by the spatial candidates (bit-identical lists), each timed with HIP events on
    the launch stream (GPU time of the screening calls) and by the wall clock."""
    import numpy as np
    import torch
    import __graft_entry__ as ge

    g = ge.load_package()
    import importlib
    wl = importlib.import_module("gs_dft_amd.workloads")
    from gs_dft_amd import _lib

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    if args.system == 6:
        s = wl.make_globule2100(**({} if args.eps is None else {"eps": args.eps}))
    else:
        s = wl.make_system(args.system, **({} if args.eps is None else {"eps": args.eps}))
    M = s.M
    log(f"{s.name}: M={M} eps={s.eps} unique={s.unique}")
    mk = lambda a: torch.tensor(a, device=dev, dtype=torch.float64)
    basis = g.Splat(quat=mk(s.quat), log_scale=mk(s.log_scale), centers=mk(s.centers))
    _lib.profile_enable(True)
    res = {}
    lists = {}
    for name, sp in (("dense", False), ("spatial", True)):
        for _ in range(args.warmup):
            g.neighbor_pairs(basis, eps=s.eps, unique=s.unique, spatial=sp)
        torch.cuda.synchronize()
        _lib.profile_read(_lib.PROF_SCREEN, reset=True)
        t0 = time.perf_counter()
        for _ in range(max(args.steps, 1)):
            lists[name] = g.neighbor_pairs(basis, eps=s.eps, unique=s.unique, spatial=sp)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / max(args.steps, 1)
        gpu_ms, calls = _lib.profile_read(_lib.PROF_SCREEN, reset=True)
        res[name] = {"wall_ms": wall * 1e3, "gpu_ms": gpu_ms / max(args.steps, 1),
                     "calls_per_build": calls / max(args.steps, 1)}
        log(f"{name}: {res[name]['wall_ms']:.2f} ms wall, {res[name]['gpu_ms']:.2f} ms in the "
            f"screening calls (count + build)")
    _lib.profile_enable(False)
    same = all(torch.equal(a, b) for a, b in zip(lists["dense"], lists["spatial"]))
    n = int(lists["dense"][0].shape[0])
    cand = M * (M + 1) // 2 if s.unique else M * M
    out = {
        "metric": "pair-list build wall ms (count + build), dense scan vs spatial candidates",
        "value": res["spatial"]["wall_ms"], "unit": "ms per pair-list build (spatial)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": res["spatial"]["wall_ms"], "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f64", "data": "synthetic",
        "config": {"workload": f"{s.name}: significant-pair list, M={M} splats, eps={s.eps}, "
                               f"unique pairs", "M": M, "eps": s.eps, "n_pairs": n,
                   "candidates": cand, "parallelism": "single GPU"},
        "dense": res["dense"], "spatial": res["spatial"], "identical_lists": bool(same),
        "speedup": res["dense"]["gpu_ms"] / max(res["spatial"]["gpu_ms"], 1e-9),
    }
    print(json.dumps(_with_command(out)), flush=True)
    return 0 if same else 1


if __name__ == "__main__":
    sys.exit(main())
