import sys

from mround_amd.cli import main

sys.exit(main())
