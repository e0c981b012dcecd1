"""TEST INFRASTRUCTURE ONLY: the CPU checker (see oracle.py). Not importable from the product."""
