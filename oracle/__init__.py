"""CPU oracle of the ntops hot path -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
package, and only as the checker; ntops_amd never imports it."""

from oracle import ops

__all__ = ["ops"]
