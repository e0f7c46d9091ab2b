"""Imports the product package (its directory name is not an identifier)."""
import importlib
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

smq = importlib.import_module("smolmoe-c99_amd")
synth = importlib.import_module("smolmoe-c99_amd.synth")
smoe = importlib.import_module("smolmoe-c99_amd.smoe")
smodel = importlib.import_module("smolmoe-c99_amd.model")
