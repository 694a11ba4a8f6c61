"""``python -m kernelforge`` runs the CLI."""

from kernelforge.cli.main import main

raise SystemExit(main())
