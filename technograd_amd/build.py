"""Compile the backend (and, for tests, the CPU oracle) in-tree."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def build(force=True, oracle=True):
    jobs = ["-j8"]
    subprocess.run(["make"] + (["-B"] if force else []) + jobs + ["-C", HERE], check=True)
    if oracle:
        targets = ["all"]
        if os.path.isdir("/root/reference/src"):
            targets.append("ref")  # the reference build exists only where its sources are
        subprocess.run(["make"] + (["-B"] if force else []) + jobs + ["-C", os.path.join(ROOT, "oracle")] + targets, check=True)
