"""The collected test count of every test file equals tests/expected_test_counts.txt, so no test
disappears (or appears) without the manifest saying so -- the role of the reference's
test/expected_test_counts.txt checked by tools/check_test_counts.sh:1-25."""
import collections
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MANIFEST = os.path.join(ROOT, "tests", "expected_test_counts.txt")


def _expected():
    out = {}
    with open(MANIFEST) as f:
        for line in f:
            line = line.strip()
            if line and not line.startswith("#"):
                path, n = line.split()
                out[path] = int(n)
    return out


def _collected():
    r = subprocess.run([sys.executable, "-m", "pytest", "tests", "--collect-only", "-q", "-p", "no:cacheprovider"],
                       cwd=ROOT, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    counts = collections.Counter(line.split("::", 1)[0] for line in r.stdout.splitlines() if "::" in line)
    return dict(counts)


def test_collected_counts_match_manifest():
    exp, got = _expected(), _collected()
    missing = {k: v for k, v in exp.items() if got.get(k, 0) != v}
    extra = {k: v for k, v in got.items() if k not in exp}
    assert not missing and not extra, (
        "collected test counts differ from tests/expected_test_counts.txt: expected "
        f"{ {k: exp[k] for k in missing} } got { {k: got.get(k, 0) for k in missing} }; files not in the manifest: {extra}")


def test_bench_refuses_several_gpus():
    """bench.py measures one GPU; asked for more it exits non-zero with a message saying so."""
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], cwd=ROOT, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
