"""Loader of the committed golden fixtures (tests/golden/*.json)."""
import json
import os

_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name: str) -> dict:
    with open(os.path.join(_DIR, f"{name}.json")) as f:
        return json.load(f)
