"""Print a GGUF file's tensors and metadata: the si-gguf-inspect tool
(src/bin/si-gguf-inspect.rs:1-102) over the C store.

    python -m si_hip.gguf_inspect --model PATH

Exit status 0 after the dump, 1 with "error: <message>" on stderr when the
file does not open or parse, 2 with the usage line for bad arguments."""
from __future__ import annotations

import sys

from . import GgufFile, HipError


def parse_model(arguments: list[str]) -> str | None:
    """Only `--model PATH` pairs are accepted; the last one wins
    (si-gguf-inspect.rs:71-83)."""
    model = None
    i = 0
    while i < len(arguments):
        if arguments[i] != "--model":
            return None
        model = arguments[i + 1] if i + 1 < len(arguments) else None
        i += 2
    return model


def main(argv: list[str] | None = None) -> int:
    model = parse_model(sys.argv[1:] if argv is None else argv)
    if model is None:
        print("Usage: si-gguf-inspect --model PATH", file=sys.stderr)
        return 2
    try:
        store = GgufFile(path=model)
    except HipError as e:
        print(f"error: {e.message}", file=sys.stderr)
        return 1
    with store:
        print(store.inspect(model))
    return 0


if __name__ == "__main__":
    sys.exit(main())
