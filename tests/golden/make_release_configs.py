"""Writes tests/golden/release_configs.json: the two config layouts the release ships
(docs/reference/config.json, the flat inference file, and docs/reference/hub_config.json, the
HF hub file with its nested text_config), stored verbatim as data for the ModelArgs tests.

Run in the container that holds the reference tree:  python tests/golden/make_release_configs.py
"""

import json
import os

REF = "/root/reference/docs/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "release_configs.json")


def main():
    with open(os.path.join(REF, "config.json")) as f:
        flat = json.load(f)
    with open(os.path.join(REF, "hub_config.json")) as f:
        hub = json.load(f)
    with open(OUT, "w") as f:
        json.dump({"flat": flat, "hub": hub}, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
