"""``python -m kernelo_amd`` runs the CLI."""

from kernelo_amd.cli.main import main

raise SystemExit(main())
