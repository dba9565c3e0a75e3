"""The apply kernel divides by a block magnitude through its reciprocal plus one
fma correction (gefenx_device.h div_by_block).  The index bit-exactness depends
on that being the correctly rounded quotient; this compiles the same sequence
for the host (gcc, glibc fmaf) and compares it with IEEE division on ~20M
pairs from the kernel's domain (|u| <= b); then div_by_const (the same step
for the factored stepsize's divisions by mean(v_row) and bc2, with under- and
overflow guards) on ~20M pairs whose quotients range far above and below 1."""
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))


def test_reciprocal_division_is_correctly_rounded():
    src = os.path.join(HERE, "c", "division_identity.c")
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "div_check")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", exe, src, "-lm"],
                       check=True)
        res = subprocess.run([exe, "20000000"], capture_output=True, text=True)
    bad, checked = (int(x) for x in res.stdout.split())
    assert checked > 20000000
    assert bad == 0, res.stderr
