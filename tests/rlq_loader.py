"""Import the product package (directory `rust-llama_amd`, not a Python
identifier) for the tests."""
import importlib
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def load():
    return importlib.import_module("rust-llama_amd")
