"""The SERVICE program's start-up checks, on the CPU: it is built next to
the library, links against it, and refuses to start without SERVICE=1 or
without a readable checkpoint (picchio.c main: usage and config errors go to
stderr with exit status 1, nothing on stdout)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "picchio_amd", "picchio_service")


@pytest.fixture(scope="module")
def service_bin():
    if not os.path.exists(BIN):
        from picchio_amd import build
        build.build_service()
    return BIN


def _run(env_extra, args=()):
    env = {k: v for k, v in os.environ.items() if k not in ("SERVICE", "MODEL")}
    env.update(env_extra)
    return subprocess.run([BIN, *args], env=env, input=b"", capture_output=True, timeout=60)


def test_needs_service_mode(service_bin, tmp_path):
    r = _run({"MODEL": str(tmp_path)})
    assert r.returncode == 1 and r.stdout == b"" and b"SERVICE=1" in r.stderr


def test_needs_a_checkpoint(service_bin, tmp_path):
    r = _run({"SERVICE": "1", "MODEL": str(tmp_path / "missing")})
    assert r.returncode == 1 and r.stdout == b"" and b"error" in r.stderr
    r = _run({"SERVICE": "1"})
    assert r.returncode == 1 and r.stdout == b""
