"""bench.py's contract on a CPU-only host: more than one GPU is refused with
a JSON message before anything touches a device, and the synthetic search
roots are legal, unfinished games of the requested length."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_search_roots_are_legal_unfinished_games():
    sys.path.insert(0, ROOT)
    import bench
    from oracle import movegen

    games = bench.search_games(4, plies=30, seed=3)
    assert len(games) == 4
    for g in games:
        assert len(g.moves) == 30 and len(g.moves_seconds) == 30
        b = movegen.board_after(g.moves)  # the Python rules replay every move as legal
        assert b.outcome() is None and g.legal_moves == b.legal_uci()
