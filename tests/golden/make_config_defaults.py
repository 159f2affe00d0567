"""Write the reference `GPAConfig` field defaults to tests/golden/config_defaults.json.

Run in the build container only (the reference is not present elsewhere):

    python tests/golden/make_config_defaults.py

The reference source (src/gpa/attention.py, `class GPAConfig`) is parsed as
text with `ast`; nothing is imported or executed.  The fixture lists every
field in declaration order with its default value.
"""
from __future__ import annotations

import ast
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCE = "/root/reference/src/gpa/attention.py"


_OPS = {ast.Div: lambda a, b: a / b, ast.Mult: lambda a, b: a * b,
        ast.Add: lambda a, b: a + b, ast.Sub: lambda a, b: a - b}


def constant(node):
    """The value of a literal, or of arithmetic on literals (e.g. 1 / 16)."""
    if isinstance(node, ast.BinOp) and type(node.op) in _OPS:
        return _OPS[type(node.op)](constant(node.left), constant(node.right))
    return ast.literal_eval(node)


def main() -> None:
    with open(SOURCE) as f:
        tree = ast.parse(f.read())
    cls = next(n for n in tree.body if isinstance(n, ast.ClassDef) and n.name == "GPAConfig")
    fields = []
    for node in cls.body:
        if isinstance(node, ast.AnnAssign) and isinstance(node.target, ast.Name):
            value = constant(node.value)
            fields.append([node.target.id, list(value) if isinstance(value, tuple) else value])
    with open(os.path.join(HERE, "config_defaults.json"), "w") as f:
        json.dump({"source": "src/gpa/attention.py GPAConfig", "fields": fields}, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
