"""Fixture from a checkpoint the reference ships (checkpoints/ckpt_00500.bin,
written by its model_save, src/transformer.c:573-616): the 56 header bytes
(magic and ModelConfig) and the file size, for the checkpoint-layout tests
to check the section arithmetic against without the reference present.

Run where the reference is present: python tests/golden/make_ckpt_fixture.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = "/root/reference/checkpoints/ckpt_00500.bin"


def main():
    if not os.path.exists(SRC):
        sys.exit(f"{SRC} missing")
    with open(SRC, "rb") as f:
        header = f.read(56)
    np.savez_compressed(os.path.join(HERE, "ckpt_reference_header.npz"),
                        header=np.frombuffer(header, np.uint8), size=os.path.getsize(SRC))


if __name__ == "__main__":
    main()
