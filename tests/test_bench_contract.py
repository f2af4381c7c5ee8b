"""bench.py's contract on the CPU: its single-GPU guard, and the HBM-traffic
figure it reports for the headline kernel. That figure comes from a committed
rocprof summary and is used only while the summary's source digest equals the
digest of the current kernel sources, so a kernel change without a new profile
would silently turn `roofline.traffic` into null; these tests catch that here."""
from __future__ import annotations

import re
import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]
PROFILE = ROOT / "profiles" / "attention_bf16_s73984_traffic.md"


def test_traffic_profile_matches_the_current_kernel_sources():
    t = bench.profiled_traffic()
    src = t["traffic_source"]
    assert not src["stale"], f"profile digest {src['profile_csrc_digest']} != sources {src['csrc_digest']}"
    assert isinstance(t["traffic"], int) and t["traffic"] > 0


def test_traffic_figure_follows_from_the_profiles_counters():
    """hbm_bytes_per_launch = FETCH_SIZE KiB x 1024 x 2 + WRITE_SIZE KiB x 1024
    (the calibration factors the profile states), and it is at least the
    algorithmic bytes of one launch (q, k, v read and o written once)."""
    text = PROFILE.read_text()
    m = re.search(r"FETCH_SIZE ([\d,]+) KiB,\s+WRITE_SIZE ([\d,]+) KiB", text)
    assert m, "per-launch counter line not found"
    fetch_kib, write_kib = (int(g.replace(",", "")) for g in m.groups())
    assert re.search(r"factor 2\.000\).*factor 1\.000\)", text, re.S), "calibration factors changed"
    hbm = int(re.search(r"^hbm_bytes_per_launch:\s*(\d+)", text, re.M).group(1))
    assert hbm == fetch_kib * 1024 * 2 + write_kib * 1024
    algorithmic = 4 * 1 * 14 * 73984 * 128 * 2
    assert hbm >= algorithmic


def test_source_digest_ignores_comments_and_layout(tmp_path, monkeypatch):
    """The digest covers code only: a changed comment or re-indented line keeps
    it, a changed token does not."""
    csrc = tmp_path / "minimaxh3_on_k100-ai_amd" / "csrc"
    csrc.mkdir(parents=True)
    real = ROOT / "minimaxh3_on_k100-ai_amd" / "csrc"
    for name in ("h3_attention.hip", "h3_common.hpp"):
        (csrc / name).write_text((real / name).read_text())
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    base = bench.kernel_source_digest()
    f = csrc / "h3_attention.hip"
    f.write_text("// a new comment\n" + f.read_text().replace("\n", "\n  ", 3))
    assert bench.kernel_source_digest() == base
    f.write_text(f.read_text().replace("kBN", "kBN2", 1))
    assert bench.kernel_source_digest() != base


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""
