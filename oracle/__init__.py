"""CPU oracle for the attention hot path.  Test infrastructure only: imported by
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg, never by
the product package."""
