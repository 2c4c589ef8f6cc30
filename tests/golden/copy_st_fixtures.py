"""Copies the reference's safetensors fixtures (data only) into
tests/golden/st/: mini.safetensors with its manifest (tensor, shape, dtype,
crc32 of the bytes; qwen35-c/tests/fixtures/st/manifest.txt) and the tiny
three-layer model checkpoint model.safetensors
(qwen35-c/tests/fixtures/model/).  Run where the reference tree exists:

    python tests/golden/copy_st_fixtures.py
"""
import os
import shutil

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference/qwen35-c/tests/fixtures"
DST = os.path.join(HERE, "st")


def main():
    os.makedirs(DST, exist_ok=True)
    for src, name in ((os.path.join(REF, "st", "mini.safetensors"), "mini.safetensors"),
                      (os.path.join(REF, "st", "manifest.txt"), "mini_manifest.txt"),
                      (os.path.join(REF, "model", "model.safetensors"), "model.safetensors")):
        shutil.copyfile(src, os.path.join(DST, name))
        print("copied", name)


if __name__ == "__main__":
    main()
