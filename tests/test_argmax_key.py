"""The decode step's deferred argmax word (host-side restatement check, no
GPU): tests/cpp/test_argmax_key.cpp packs each workgroup's best (value, row)
as the LM head kernel does and folds the words with a maximum; the result
must be the row the kernels' comparison picks over the whole vocabulary
(higher value, then lower row; NaN and -inf never win) for any split into
workgroups."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_argmax_key_folds_to_the_comparison_winner():
    cpp = os.path.join(ROOT, "tests", "cpp")
    subprocess.run(["make", "-C", cpp, "test_argmax_key"], check=True, capture_output=True)
    done = subprocess.run([os.path.join(cpp, "test_argmax_key")], capture_output=True, text=True,
                          timeout=120)
    assert done.returncode == 0, done.stdout + done.stderr
    assert "0 failures" in done.stdout
