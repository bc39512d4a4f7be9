"""Writes converter_names.json: the GGUF names and metadata types the
reference's converter emits, read as text from its source (not run):
scripts/convert_siglip2_to_gguf.py -- the block tensor map (_map_block,
:154-171), the tower-level maps (_map_vision_non_block :174-192,
_map_text_non_block :195-205), the fused QKV names (:395-399), the probe
head's split Q/K/V (:472-476), the tensors kept F32 (_is_keep_f32,
:209-217) and the metadata keys with their types (_add_metadata, :306-353).

    python tests/golden/make_converter_names.py [path/to/convert_siglip2_to_gguf.py]
"""
import json
import os
import re
import sys

SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/scripts/convert_siglip2_to_gguf.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "converter_names.json")


def func_body(text, name):
    i = text.index(f"def {name}(")
    j = text.find("\n    def ", i + 1)
    j2 = text.find("\n    @staticmethod", i + 1)
    ends = [e for e in (j, j2) if e > 0]
    return text[i:min(ends) if ends else len(text)]


def dict_values(body):
    return re.findall(r'"[\w.]+":\s*"([\w.]+)"', body)


def main():
    text = open(SRC, encoding="utf-8").read()
    arch = re.search(r'^ARCH\s*=\s*"(\w+)"', text, re.M).group(1)
    block = sorted(dict_values(func_body(text, "_map_block")))
    # the fused QKV written per block: f"{tower}.blk.{idx}.attn_qkv" + .weight / .bias
    qkv = re.search(r'f"\{tower\}\.blk\.\{idx\}\.(\w+)"', text).group(1)
    block += [f"{qkv}.weight", f"{qkv}.bias"]
    vision = sorted(dict_values(func_body(text, "_map_vision_non_block")))
    text_t = sorted(dict_values(func_body(text, "_map_text_non_block")))
    # the probe head's in_proj split: f"v.head.attn_{tag}.weight" for the tags of the loop
    tags = re.findall(r'\("(\w)", \w_w, \w_b\)', text)
    for t in tags:
        vision += [f"v.head.attn_{t}.weight", f"v.head.attn_{t}.bias"]
    keep = func_body(text, "_is_keep_f32")
    keep_f32 = {
        "suffixes": re.findall(r'endswith\("([\w.]+)"\)', keep),
        "substrings": re.findall(r'"([\w.]+)" in ggml_name', keep),
        "names": re.findall(r'"([\w.]+)"', keep.split("ggml_name in (", 1)[1].split(")", 1)[0]),
    }
    meta = {}
    for typ, key in re.findall(r'w\.add_(uint32|float32|string|bool|array)\(f"\{ARCH\}\.([\w.]+)"',
                               text):
        meta[f"{arch}.{key}"] = typ
    out = {"source": "scripts/convert_siglip2_to_gguf.py", "arch": arch,
           "block_tensors": sorted(block), "vision_tensors": sorted(vision),
           "text_tensors": sorted(text_t), "keep_f32": keep_f32, "metadata": meta}
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print(OUT)


if __name__ == "__main__":
    main()
