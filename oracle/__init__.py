"""CPU oracle for the mHC hot path.  Test infrastructure only: imported by
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg,
never by the ``mhc_mlx_amd`` package."""
