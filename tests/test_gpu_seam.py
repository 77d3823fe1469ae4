"""The C++ host side (vibe_compiler_amd/seam): HipTargetModelBackend driven
through the reference's TargetModelOneDNNBackend / TargetModelManagedReference
Backend seams by tests/seam/seam_check.cpp, every result byte compared with
the CPU oracle packed into the same destination template."""
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
CHECK = ROOT / "tests" / "seam" / "_build" / "seam_check"


@pytest.mark.gpu
def test_seam_requests_match_oracle():
    assert CHECK.exists(), "build first: make -C tests/seam"
    print("seam_check", flush=True)
    r = subprocess.run([str(CHECK)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASSED" in r.stdout


QUALIFY = ROOT / "tests" / "seam" / "_build" / "qualify_check"


@pytest.mark.gpu
def test_qualification_records(tmp_path):
    """Evidence records (vibe_compiler_amd/seam/qualification.h): validation
    writes a record only for output bytes equal to the formal lane's; the
    verified record qualifies exactly its problem on exactly its environment;
    tampered records, other payloads and other environments are refused."""
    assert QUALIFY.exists(), "build first: make -C tests/seam"
    print("qualify_check", flush=True)
    r = subprocess.run([str(QUALIFY), str(tmp_path)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL OK" in r.stdout
