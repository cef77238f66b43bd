"""``python -m nnunet_mlx predict ...`` (see ``nnunet_mlx.cli``)."""

import sys

from nnunet_mlx.cli import main

sys.exit(main())
