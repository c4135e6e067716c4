"""python -m deciax_amd.serve — the `/v1/systemone` server on the HIP decision path.

The options and their environment fallbacks are those of the reference's CLI
(src/deciax/serve/__main__.py:34-75): DECIAX_HOST, DECIAX_PORT, DECIAX_MODELS,
DECIAX_DEFAULT_MODEL, DECIAX_MAX_CONCURRENT, DECIAX_JEV_STRICT, DECIAX_DTYPE, DECIAX_IMPL,
DECIAX_LOG_LEVEL, DECIAX_API_KEY. `--impl` takes the reference's choices plus `hip`, the value
this package serves; `--model` takes a registered shape or a checkpoint directory.
"""

from __future__ import annotations

import argparse
import logging
import os
from pathlib import Path
from typing import get_args

from deciax_amd.backend import ImplChoice
from deciax_amd.decider import DtypeChoice
from deciax_amd.gemma import CONFIGS

IMPLS: tuple[str, ...] = get_args(ImplChoice)
DTYPES: tuple[str, ...] = get_args(DtypeChoice)


def _flag(name: str) -> bool:
    return os.environ.get(name, "").strip().lower() in ("1", "true", "yes", "on")


def _model(value: str) -> str:
    if value in CONFIGS or Path(value).is_dir():
        return value
    raise argparse.ArgumentTypeError(f"unknown model {value!r}: choose one of {sorted(CONFIGS)} or a checkpoint "
                                     "directory")


def parser() -> argparse.ArgumentParser:
    env = os.environ.get
    p = argparse.ArgumentParser(prog="python -m deciax_amd.serve", description=__doc__)
    p.add_argument("--host", default=env("DECIAX_HOST", "127.0.0.1"))
    p.add_argument("--port", type=int, default=int(env("DECIAX_PORT", "8000")))
    p.add_argument("--model", action="append", dest="models", type=_model,
                   help="model to load (repeatable; default DECIAX_MODELS or gemma2-9b)")
    p.add_argument("--default-model", default=env("DECIAX_DEFAULT_MODEL"))
    p.add_argument("--max-concurrent", type=int, default=int(env("DECIAX_MAX_CONCURRENT", "16")))
    p.add_argument("--jev-strict", action="store_true", default=_flag("DECIAX_JEV_STRICT"))
    p.add_argument("--no-warmup", action="store_true")
    p.add_argument("--dtype", default=env("DECIAX_DTYPE", "auto"))
    p.add_argument("--impl", default=env("DECIAX_IMPL", "auto"))
    p.add_argument("--seed", type=int, default=0, help="weight seed of the registered random-init shapes")
    p.add_argument("--log-level", default=env("DECIAX_LOG_LEVEL", "info"))
    return p


def parse(argv: list[str] | None = None) -> argparse.Namespace:
    """Parsed options, with the choices checked on values that came from the environment too."""
    p = parser()
    args = p.parse_args(argv)
    for flag, value, choices in (("--dtype", args.dtype, DTYPES), ("--impl", args.impl, IMPLS)):
        if value not in choices:
            p.error(f"{flag}: invalid choice {value!r} (choose from {', '.join(choices)})")
    if not args.models:
        args.models = [m.strip() for m in os.environ.get("DECIAX_MODELS", "gemma2-9b").split(",") if m.strip()]
        for m in args.models:
            try:
                _model(m)
            except argparse.ArgumentTypeError as e:
                p.error(f"--model: {e}")
    if args.default_model and args.default_model not in [Path(m).name if Path(m).is_dir() else m
                                                         for m in args.models]:
        p.error(f"--default-model {args.default_model!r} is not among the loaded models")
    return args


def main(argv: list[str] | None = None) -> None:
    args = parse(argv)
    logging.basicConfig(level=args.log_level.upper(), format="%(asctime)s %(levelname)s %(name)s: %(message)s")
    from deciax_amd.serve.wsgi import serve

    serve(args.host, args.port, tuple(args.models), default_model=args.default_model or None,
          api_key=os.environ.get("DECIAX_API_KEY") or None, max_concurrent=args.max_concurrent,
          jev_strict=args.jev_strict, warmup=not args.no_warmup, dtype=args.dtype, impl=args.impl, seed=args.seed)


if __name__ == "__main__":
    main()
