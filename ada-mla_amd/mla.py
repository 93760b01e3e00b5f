"""Entry script of the MLA decode harness (the counterpart of the reference's
mla.py): `python ada-mla_amd/mla.py --test -s 4096 -k fused`. The harness
itself is ada_mla/cli.py."""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from ada_mla.cli import main  # noqa: E402

if __name__ == "__main__":
    sys.exit(main())
