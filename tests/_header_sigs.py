"""Parse include/kdn.h into {function: argument-code string} (codes as in lit_gpt/kdn_ops/_lib.py)."""
import pathlib
import re

HEADER = pathlib.Path(__file__).resolve().parent.parent / "include" / "kdn.h"


def _code(arg: str) -> str:
    arg = arg.strip()
    if arg in ("void", ""):
        return ""
    if "*" in arg:
        return "p"
    if arg.startswith("hipStream_t"):
        return "s"
    if arg.startswith("int64_t"):
        return "l"
    if arg.startswith("int"):
        return "i"
    if arg.startswith("float"):
        return "f"
    if arg.startswith("size_t"):
        return "z"
    raise ValueError(f"unknown argument type: {arg!r}")


def header_signatures() -> dict:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    sigs = {}
    for m in re.finditer(r"\b(int|size_t)\s+(kdn_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, args = m.groups()
        sigs[name] = (ret, "".join(_code(a) for a in args.split(",")))
    return sigs


if __name__ == "__main__":
    for k, (r, s) in header_signatures().items():
        print(f'    "{k}": "{s}",  # {r}')
