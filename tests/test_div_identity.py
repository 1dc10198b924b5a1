"""Exhaustive host check of the quantizers' bf16 arithmetic (tests/csrc/div_identity.c).

For every bf16 amax the refined scale must equal IEEE amax/448, and for
every bf16 x with |x| <= amax the refined divide must give the same e4m3fn
byte as the IEEE quotient, and the same f32 quotient wherever
|x/s| > 2^-10.  The sweep is split over 8 processes.
"""
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))


def test_divide_identity_all_bf16_pairs():
    src = os.path.join(HERE, "csrc", "div_identity.c")
    exe = os.path.join(tempfile.mkdtemp(), "div_identity")
    subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
    # split the amax range so each process sees a similar number of pairs (~ amax^2)
    hi = 0x7F7F
    edges = [int(hi * (k / 8) ** 0.5) for k in range(9)]
    procs = []
    for k in range(8):
        lo, up = edges[k] + (1 if k else 0), edges[k + 1]
        procs.append(subprocess.Popen([exe, hex(lo), hex(up)], stdout=subprocess.PIPE, text=True))
    pairs = enc = above = scale = 0
    for p in procs:
        out, _ = p.communicate()
        assert p.returncode == 0
        a, b, c, _, e = (int(v) for v in out.split())
        pairs, enc, above, scale = pairs + a, enc + b, above + c, scale + e
    assert pairs == sum(2 * (ab + 1) for ab in range(hi + 1))
    assert scale == 0
    assert enc == 0
    assert above == 0
