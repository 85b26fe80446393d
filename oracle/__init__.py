"""ORACLE — TEST INFRASTRUCTURE ONLY (see oracle.py). Never imported by the product path."""
