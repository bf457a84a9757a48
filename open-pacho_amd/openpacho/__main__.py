"""``python -m openpacho``: the ``pacho`` command."""

from .cli import main

raise SystemExit(main())
