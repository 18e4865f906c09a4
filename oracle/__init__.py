"""ORACLE -- test infrastructure, not product code.

CPU restatement of the reference Vesta interpreter and GPT-2 decode protocol,
used only as the checker by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``. Nothing on the GPU path imports it.
"""
