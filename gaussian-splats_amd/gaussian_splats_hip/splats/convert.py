"""Checkpoint <-> PLY conversion commands (reference:
src/gaussian_splats/splats/convert.py:1-34).

``python -m gaussian_splats_hip.splats.convert pt-to-ply scene.pt [-o scene.ply]``
and ``ply-to-pt scene.ply [-o scene.pt]``.  With ``--device cuda`` the records
are split or packed on the GPU (``load_ply(..., device=...)``, ``save_ply`` of
GPU tensors)."""

from __future__ import annotations

from pathlib import Path
from typing import Annotated, Optional

import typer

from .ply import load_ply, save_ply
from .splats import GaussianSplat

app = typer.Typer(add_completion=False, no_args_is_help=True)

_Device = Annotated[Optional[str], typer.Option("--device", help="torch device for the records")]


@app.command("pt-to-ply")
def pt_to_ply(
    checkpoint: Annotated[Path, typer.Argument(exists=True, dir_okay=False)],
    output: Annotated[Optional[Path], typer.Option("--output", "-o")] = None,
    device: _Device = None,
) -> None:
    output = output or checkpoint.with_suffix(".ply")
    splats = GaussianSplat.from_checkpoint(checkpoint)
    if device is not None:
        splats = splats.to(device)
    save_ply(splats.state_dict(), output)
    typer.echo(f"Wrote {output}")


@app.command("ply-to-pt")
def ply_to_pt(
    checkpoint: Annotated[Path, typer.Argument(exists=True, dir_okay=False)],
    output: Annotated[Optional[Path], typer.Option("--output", "-o")] = None,
    device: _Device = None,
) -> None:
    output = output or checkpoint.with_suffix(".pt")
    GaussianSplat.from_tensors(**load_ply(checkpoint, device=device)).save_checkpoint(output)
    typer.echo(f"Wrote {output}")


if __name__ == "__main__":
    app()
