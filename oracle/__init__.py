"""CPU oracle (test infrastructure only): see oracle/oracle.py and oracle/model.py."""
