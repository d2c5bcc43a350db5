"""CPU oracle (test infrastructure only): see ``fourbit_oracle``.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package.  The product package ``if_i_could_turn_back_time_amd`` never does.
"""
