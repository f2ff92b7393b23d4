"""The softmax's ggml_v_expf with the x <= 0 specialisation gives the general
function's bits (i2s_device.h: NONPOS). Host C, both forms as the
device computes them; a stride through every float with the sign bit set,
plus the exponent boundaries of the range selects, plus sampled NaNs. (The
whole 2^31 run matches too; it takes minutes.)"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def test_nonpositive_expf_matches_the_general_one(tmp_path):
    exe = tmp_path / "expf_nonpos"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), os.path.join(HERE, "native", "expf_nonpos.c"),
                    "-lm"], check=True)
    r = subprocess.run([str(exe), "257"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 differ" in r.stdout
