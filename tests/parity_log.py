"""Parity records the GPU tests leave for the end of the run: every attention
comparison made through mla_bar.check_bar (observed max-abs, mean-abs,
elements over the flat 2e-2 bar and whether the two-ulp exception for
|ref| >= 2 was needed) and the exact comparisons of the cache writer and
the MoE aligner.  Comparisons on the five benchmark configurations carry a
config label; tests/conftest.py prints one line per label and lists every
comparison that needed the exception, so the magnitudes reach the summary
of a plain `pytest -q` run."""
import os

ATTENTION = []
EXACT = []

CONFIGS = {
    "rows16384_b1": "16384-row cache, B=1, 2048 uniform + 128 pads",
    "moe_align_b1_b8": "MoE align, distinct top-8 and shared top-8, B in {1,2,4,8}",
    "rows262144_normal_b1": "262144-row N(0,1) cache, B=1, 2048 uniform + 128 pads",
    "rows262144_t3_b8": "262144-row Student-t cache, B=8, locality-biased, 0-256 pads",
    "prefill_t2048": "prefill-shaped T=2048 over the Student-t cache; 2048 scattered writes",
}


def current_test():
    return os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]


def record_attention(tag, config, max_abs, mean_abs, n_over, n, worst_ulp, max_abs_bar, mean_abs_bar):
    ATTENTION.append(dict(test=current_test(), tag=str(tag), config=config, max_abs=max_abs, mean_abs=mean_abs,
                          n_over=n_over, n=n, worst_ulp=worst_ulp,
                          literal=max_abs <= max_abs_bar and mean_abs <= mean_abs_bar))


def record_exact(config, what, differing, total):
    EXACT.append(dict(test=current_test(), config=config, what=what, differing=int(differing), total=int(total)))


def summary_lines():
    lines = []
    if not ATTENTION and not EXACT:
        return lines
    lines.append("parity bars: bf16 attention max-abs <= 2e-2 and mean-abs <= 2e-3 against the oracle; "
                 "cache rows and MoE align outputs bit-exact")
    for cfg, desc in CONFIGS.items():
        ex = [r for r in EXACT if r["config"] == cfg]
        at = [r for r in ATTENTION if r["config"] == cfg]
        for what in dict.fromkeys(r["what"] for r in ex):
            rs = [r for r in ex if r["what"] == what]
            lines.append(f"{cfg} {what}: {sum(r['differing'] for r in rs)} of {sum(r['total'] for r in rs)} "
                         f"differ ({len(rs)} comparisons)")
        if at:
            over = sum(r["n_over"] for r in at)
            n = sum(r["n"] for r in at)
            lines.append(f"{cfg} attention ({desc}): {len(at)} comparisons, max-abs "
                         f"{max(r['max_abs'] for r in at):.4g}, mean-abs {max(r['mean_abs'] for r in at):.3g} (worst), "
                         f"{over} of {n} elements over 2e-2, literal bar held by {sum(r['literal'] for r in at)}")
    if ATTENTION:
        held = sum(r["literal"] for r in ATTENTION)
        lines.append(f"all attention comparisons: {len(ATTENTION)}; the literal bar (flat max-abs 2e-2, mean-abs "
                     f"2e-3) held by {held}; the rest needed the exception (|ref| >= 2, within 2 bf16 ulps, at "
                     f"most max(2, n / 1e5) elements):")
        for r in ATTENTION:
            if not r["literal"]:
                lines.append(f"  {r['test']} [{r['tag']}]: max-abs {r['max_abs']:.4g}, {r['n_over']} of {r['n']} "
                             f"elements over 2e-2, at most {r['worst_ulp']:.2g} bf16 ulp")
    return lines
