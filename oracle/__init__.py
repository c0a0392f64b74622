"""CPU oracle for the KDA chunkwise recurrence -- TEST INFRASTRUCTURE ONLY.

Everything under ``oracle/`` restates the reference's algorithm on the CPU so
that the HIP path can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import, call or link anything here, and only as the checker (or the timed CPU
baseline), never as part of the product path.  ``mlx_vit_amd`` never imports
this package; when its HIP library is missing it raises instead of falling
back to anything in here.

Modules
-------
``kda_reference``  torch restatement (any float dtype) of the reference's
                   step recurrence, its chunkwise WY algebra, both backwards,
                   the triangular solves, and the benchmark input generator.
``kda_oracle.c``   plain-C fp64 restatement of the step recurrence (rank-1
                   form) with its reverse-time backward; multithreaded over
                   (batch, head) so full-size configs finish in seconds.
``cref``           ctypes binding for the C oracle (``liboracle_kda.so``).
"""
