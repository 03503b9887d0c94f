"""Writes tests/golden/vocab.json from the reference move table.

The reference table (src/modeling/moves.py:3-1972) is read as TEXT with
``ast.literal_eval`` -- nothing of the reference is imported or executed.
The fixture keeps only a SHA-256 of the newline-joined list, its length and
a sample of (index, move) pairs; the engine generates the table itself
(allie_amd/vocab.py) and tests/test_vocab.py checks it against this file.

Run in a container that has /root/reference:
    python tests/golden/make_vocab_golden.py
"""
import ast
import hashlib
import json
import os

REF = "/root/reference/src/modeling/moves.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "vocab.json")


def main() -> None:
    tree = ast.parse(open(REF).read())
    moves = None
    for node in tree.body:
        if isinstance(node, ast.Assign) and getattr(node.targets[0], "id", "") == "CHESS_MOVES":
            moves = ast.literal_eval(node.value)
    assert moves is not None
    idx = sorted(set(list(range(0, len(moves), 97)) + [1, 2, 1455, 1456, 1795, 1796, 1966, 1967]))
    out = {
        "source": "src/modeling/moves.py:3-1972 (read as text)",
        "count": len(moves),
        "sha256_newline_joined": hashlib.sha256("\n".join(moves).encode()).hexdigest(),
        "samples": {str(i): moves[i] for i in idx},
    }
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
