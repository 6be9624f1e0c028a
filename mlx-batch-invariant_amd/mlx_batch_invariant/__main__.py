"""`python -m mlx_batch_invariant verify` -- same as the `mlx-bi` console script."""
import sys

from ._cli import main

sys.exit(main())
