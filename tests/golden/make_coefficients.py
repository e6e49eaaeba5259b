"""Write tests/golden/coefficients.json: the reference's Newton-Schulz tables.

Reads the reference's source files as text and evaluates only the literal
assignments of its coefficient tables (nothing is imported or run):
``_GRAM_SAFETY`` and ``_GRAM_UNMODIFIED`` (src/dionw/_gram.py:24-31),
``GRAM_RESTART_ITERATION`` (:37), ``POLAR_EXPRESS_COEFFICIENTS`` and
``POLAR_EXPRESS_NORM_SAFETY`` (_polar_express.py:28-36),
``KELLER_COEFFICIENTS`` and ``KELLER_NORM_SAFETY`` (_keller.py:20-22).

Usage: python tests/golden/make_coefficients.py [/path/to/reference]
"""

from __future__ import annotations

import ast
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
NAMES = {
    "_gram.py": ("_GRAM_SAFETY", "_GRAM_UNMODIFIED", "GRAM_RESTART_ITERATION"),
    "_polar_express.py": ("POLAR_EXPRESS_COEFFICIENTS", "POLAR_EXPRESS_NORM_SAFETY"),
    "_keller.py": ("KELLER_COEFFICIENTS", "KELLER_NORM_SAFETY"),
}


def _value(node: ast.expr):
    """A literal, or a literal tuple repeated (``(row,) * 5``)."""
    if isinstance(node, ast.BinOp) and isinstance(node.op, ast.Mult):
        return tuple(_value(node.left)) * _value(node.right)
    return ast.literal_eval(node)


def extract(reference: Path) -> dict:
    found = {}
    for name, wanted in NAMES.items():
        tree = ast.parse((reference / "src" / "dionw" / name).read_text())
        for stmt in tree.body:
            if isinstance(stmt, ast.AnnAssign) and isinstance(stmt.target, ast.Name):
                target, value = stmt.target.id, stmt.value
            elif isinstance(stmt, ast.Assign) and isinstance(stmt.targets[0], ast.Name):
                target, value = stmt.targets[0].id, stmt.value
            else:
                continue
            if target in wanted and value is not None:
                found[target] = _value(value)
    missing = {n for names in NAMES.values() for n in names} - set(found)
    if missing:
        raise SystemExit(f"not found in the reference: {sorted(missing)}")
    return {
        "gram_safety": found["_GRAM_SAFETY"],
        "gram_unmodified": [list(r) for r in found["_GRAM_UNMODIFIED"]],
        "gram_restart_iteration": found["GRAM_RESTART_ITERATION"],
        "polar_express": [list(r) for r in found["POLAR_EXPRESS_COEFFICIENTS"]],
        "polar_express_norm_safety": found["POLAR_EXPRESS_NORM_SAFETY"],
        "keller": [list(r) for r in found["KELLER_COEFFICIENTS"]],
        "keller_norm_safety": found["KELLER_NORM_SAFETY"],
    }


def main() -> None:
    reference = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
    out = HERE / "coefficients.json"
    out.write_text(json.dumps(extract(reference), indent=1) + "\n")
    print("wrote", out)


if __name__ == "__main__":
    main()
