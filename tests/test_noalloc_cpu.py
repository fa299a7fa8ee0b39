"""CPU check of the allocation-free decode GEMM's entry: before
catena_mi355x_init it refuses (it never initialises the library itself,
since init allocates), without touching a device.  Runs in a child process
so that no earlier test has initialised the library."""
import os
import subprocess
import sys
import textwrap

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_noalloc_requires_init():
    code = textwrap.dedent(f"""
        import sys
        sys.path.insert(0, {os.path.join(ROOT, 'catena-lang_amd')!r})
        import catena_amd as ca
        L = ca.lib()
        st = L.catena_mi355x_gemm_bf16_decode_noalloc(16, 32, 48, 16, 128, 128, 0)
        print(st, ca.last_error())
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-500:]
    st, _, msg = r.stdout.strip().partition(" ")
    assert st == "5" and "catena_mi355x_init" in msg
