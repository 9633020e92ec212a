"""Command line: ``python -m mlx_gsq_amd.gguf {analyze,convert,verify}`` (the reference's
mlx_gsq/gguf/__main__.py:8-22 commands and options)."""
from __future__ import annotations

import argparse
from pathlib import Path

from .converter import convert_gguf_to_safetensors, verify_conversion
from .reader import write_analysis


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(prog="python -m mlx_gsq_amd.gguf")
    sub = ap.add_subparsers(dest="command", required=True)
    a = sub.add_parser("analyze", help="validate a GGUF file and write its analysis JSON")
    a.add_argument("model", type=Path)
    a.add_argument("-o", "--output", type=Path, default=Path("analysis.json"))
    c = sub.add_parser("convert", help="write the packed Safetensors container")
    c.add_argument("model", type=Path)
    c.add_argument("output", type=Path)
    c.add_argument("--overwrite", action="store_true")
    c.add_argument("--no-verify", action="store_true")
    v = sub.add_parser("verify", help="check a container against its GGUF source")
    v.add_argument("model", type=Path)
    v.add_argument("output", type=Path)
    args = ap.parse_args(argv)
    if args.command == "analyze":
        result = write_analysis(args.model, args.output)
        print(f"validated {result['summary']['total_tensors']} tensors -> {args.output}")
    elif args.command == "convert":
        out = convert_gguf_to_safetensors(args.model, args.output, overwrite=args.overwrite, verify=not args.no_verify)
        print(f"wrote {out}")
    else:
        verify_conversion(args.model, args.output)
        print("verification passed")


if __name__ == "__main__":
    main()
