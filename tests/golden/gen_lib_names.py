"""Writes tests/golden/lib_py_names.txt: the C symbol names the reference's Python bindings bind at
import (newch/_lib.py:78-177, `getattr(lib, _name)` for every key of _SIGNATURES).

The file is read as text and its _SIGNATURES literal is walked with `ast` (nothing is imported or
executed).  Run in a container that has the reference tree:

    python tests/golden/gen_lib_names.py
"""

import ast
from pathlib import Path

SRC = Path("/root/reference/newch/_lib.py")
OUT = Path(__file__).resolve().parent / "lib_py_names.txt"


def names_from_dict(node: ast.Dict) -> list[str]:
    out = []
    for key, value in zip(node.keys, node.values):
        if key is not None:
            out.append(ast.literal_eval(key))
            continue
        comp = value  # **{f"nc_{n}": ... for n in (...)}
        assert isinstance(comp, ast.DictComp), ast.dump(comp)
        fmt = comp.key
        assert isinstance(fmt, ast.JoinedStr)
        prefix = "".join(v.value for v in fmt.values if isinstance(v, ast.Constant))
        for gen in comp.generators:
            for elt in ast.literal_eval(gen.iter):
                out.append(prefix + elt)
    return out


def main():
    tree = ast.parse(SRC.read_text())
    for node in ast.walk(tree):
        if isinstance(node, ast.Assign) and any(getattr(t, "id", None) == "_SIGNATURES" for t in node.targets):
            names = names_from_dict(node.value)
            OUT.write_text("\n".join(sorted(set(names))) + "\n")
            print(f"{len(set(names))} names -> {OUT}")
            return
    raise SystemExit("_SIGNATURES not found")


if __name__ == "__main__":
    main()
