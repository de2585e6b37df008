"""``python -m harness ...``: see harness.cli."""

from .cli import main

raise SystemExit(main())
