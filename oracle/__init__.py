"""CPU oracle for the slot-scan hot path -- test infrastructure only (tests/, __graft_entry__.smoke(),
bench.py's cpu_baseline).  The product path never imports anything from here."""
