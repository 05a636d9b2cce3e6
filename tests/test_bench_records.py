"""bench.py's measured constants against the committed rocprof summaries they
come from: the HBM counter values behind the roofline's `traffic` field must
be the ones in profiles/gn_silu_fwd_bwd_n256_64x64x256.md, digit for digit,
for the kernel the bench names as its roofline kernel."""
from __future__ import annotations

import importlib.util
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PROFILE = ROOT / "profiles" / "gn_silu_fwd_bwd_n256_64x64x256.md"


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _pmc_table(text: str) -> dict[str, tuple[int, int]]:
    """Rows of the profile's 'HBM traffic per dispatch (PMC)' table:
    kernel -> (FETCH_SIZE KiB, WRITE_SIZE KiB)."""
    section = text.split("## HBM traffic per dispatch (PMC)", 1)[1].split("\n## ", 1)[0]
    rows = {}
    for m in re.finditer(r"^\| `([^`]+)` \| ([\d,]+) \| ([\d,]+) \|", section, flags=re.M):
        rows[m.group(1)] = (int(m.group(2).replace(",", "")), int(m.group(3).replace(",", "")))
    return rows


def test_roofline_traffic_constants_match_the_committed_profile():
    bench = _bench()
    rows = _pmc_table(PROFILE.read_text())
    assert bench.ROOFLINE_KERNEL in rows, (bench.ROOFLINE_KERNEL, sorted(rows))
    for kernel, counts in bench._PMC_KIB.items():
        assert rows.get(kernel) == counts, (kernel, counts, rows.get(kernel))
    fetch, write = rows[bench.ROOFLINE_KERNEL]
    assert bench.TRAFFIC_BYTES == (2 * fetch + write) * 1024


def test_profile_kernel_trace_names_the_roofline_kernel():
    bench = _bench()
    text = PROFILE.read_text()
    trace = text.split("## Kernel trace of the driver command", 1)[1].split("\n## ", 1)[0]
    assert f"`{bench.ROOFLINE_KERNEL}`" in trace
