"""CPU restatement of the reference WKV7 recurrence -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker.  The product
package never imports it.
"""
from . import int6_ref  # noqa: F401
from .wkv7_ref import build, max_threads, rel_fro, rel_max, wkv7_ref, wkv7_ref_numpy  # noqa: F401
