"""turkce-llm_amd: MI355X-native GPU matmul path of turkce-llm.

The directory name is not a Python identifier; load it with
`importlib` (see tests/conftest.py, bench.py) or import `trlm` after adding
this directory to sys.path.
"""
from .trlm import *  # noqa: F401,F403
