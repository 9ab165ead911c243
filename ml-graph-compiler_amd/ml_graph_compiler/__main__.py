"""``python -m ml_graph_compiler``: the command line interface."""

import sys

from .cli import main

sys.exit(main())
