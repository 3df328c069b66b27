"""The two commands' argument handling, without a device: `maxim_hip` (the
reference's release CLI, src/main.rs:59-158) and `python -m maxim_amd` (its
development flags). Both refuse the CPU backend and the flags they do not
have by name (exit 2), print the version, and report a missing model or an
unreadable input before touching the GPU."""

import os
import subprocess
import sys

import pytest

from conftest import ROOT

EXE = os.path.join(ROOT, "maxim-rs_amd", "lib", "maxim_hip")


def run(args, py=False):
    if py:
        env = dict(os.environ, PYTHONPATH=os.path.join(ROOT, "maxim-rs_amd"))
        cmd = [sys.executable, "-m", "maxim_amd"] + args
    else:
        env, cmd = None, [EXE] + args
    return subprocess.run(cmd, capture_output=True, text=True, timeout=120, env=env)


def test_release_command_arguments():
    r = run(["-V"])
    assert r.returncode == 0 and r.stdout.startswith("maxim_hip ")
    for args, what in [(["--cpu", "-m", "x"], "no CPU backend"), (["--device", "cpu", "-m", "x"], "no CPU backend"),
                       (["--dump", "d", "-m", "x"], "development flag"), (["--profile"], "development flag"),
                       (["--bogus"], "unknown argument"), (["-i", "a.png"], "--model is required"),
                       (["-h"], "usage:")]:
        r = run(args)
        assert r.returncode == 2 and what in r.stderr, (args, r.returncode, r.stderr)


@pytest.mark.parametrize("args,code,what", [
    (["--cpu", "-m", "x"], 2, "no CPU backend"),
    (["--verify-gpu", "-m", "x"], 2, "verify_walk"),
    (["-i", "a.png"], 2, "--model is required"),
    (["--factor", "0", "-m", "x"], 2, "--factor"),
    (["-m", "x", "-i", "/nonexistent/in.png"], 1, "/nonexistent/in.png"),
])
def test_dev_entry_point_arguments(args, code, what):
    r = run(args, py=True)
    assert r.returncode == code and what in r.stderr, (args, r.returncode, r.stderr)
