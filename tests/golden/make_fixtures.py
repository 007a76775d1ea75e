"""Writes the golden fixtures under tests/golden/ from the reference's test data.

Run here, where the reference tree is mounted; the fixtures it writes are
committed, and nothing at test time reads the reference.

For each sealed tiny bundle (testdata/tiny-bert-bundle, tiny-modernbert-bundle,
tiny-nomic-bundle) it keeps the upstream reference cases (token ids, lengths
and the fp32 vectors upstream sentence-transformers produced) and the bundle's
weights. To keep the files small, the word-embedding table keeps only the rows
the cases' ids use (and the pad row 0), in id order, and the ids are renumbered
to those rows: the same rows of the same table meet the same ids, so every
vector is unchanged. The architecture comes from the bundle's manifest.
"""
import json
import os
import sys

import numpy as np
from safetensors.numpy import load_file, save_file

REF = "/root/reference/testdata"
HERE = os.path.dirname(os.path.abspath(__file__))


def bert_order(layers):
    emb = ["word_embeddings", "position_embeddings", "token_type_embeddings", "embeddings_ln_weight",
           "embeddings_ln_bias"]
    per = ["q_weight", "q_bias", "k_weight", "k_bias", "v_weight", "v_bias", "attn_out_weight", "attn_out_bias",
           "attn_ln_weight", "attn_ln_bias", "ffn_in_weight", "ffn_in_bias", "ffn_out_weight", "ffn_out_bias",
           "ffn_ln_weight", "ffn_ln_bias"]
    return emb, per


def modernbert_order():
    return (["word_embeddings", "embeddings_ln_weight", "final_norm_weight"],
            ["attn_ln_weight", "qkv_weight", "attn_out_weight", "ffn_ln_weight", "ffn_in_weight", "ffn_out_weight"])


def nomic_order():
    return (["word_embeddings", "token_type_embeddings", "embeddings_ln_weight", "embeddings_ln_bias"],
            ["qkv_weight", "attn_out_weight", "attn_ln_weight", "attn_ln_bias", "ffn_gate_weight", "ffn_up_weight",
             "ffn_out_weight", "ffn_ln_weight", "ffn_ln_bias"])


def one(bundle, out_name):
    d = os.path.join(REF, bundle)
    m = json.load(open(os.path.join(d, "manifest.json")))
    arch = m["architecture"]
    art = m["artifacts"][0]
    names = art["tensor_names"]
    weights = load_file(os.path.join(d, art["files"][0]))
    ref = load_file(os.path.join(d, m["reference"]["file"]))
    ids, lengths, vectors = ref["ids"], ref["lengths"], ref["embeddings"]
    family = arch["family"]
    emb, per = {"FAMILY_BERT": bert_order(arch["layers"]), "FAMILY_MODERNBERT": modernbert_order(),
                "FAMILY_NOMIC_BERT": nomic_order()}[family]
    used = sorted(set(int(v) for r, n in zip(ids, lengths) for v in r[:n]) | {0})
    remap = {old: new for new, old in enumerate(used)}
    new_ids = np.zeros_like(ids)
    for i, (r, n) in enumerate(zip(ids, lengths)):
        new_ids[i, :n] = [remap[int(v)] for v in r[:n]]
    tensors = {}
    order = []
    for key in emb:
        t = weights[names[key]]
        if key == "word_embeddings":
            t = t[used]
        tensors[f"emb.{key}"] = np.ascontiguousarray(t)
        order.append(f"emb.{key}")
    for layer in range(arch["layers"]):
        for key in per:
            name = names[key].replace("{layer}", str(layer))
            if name not in weights:      # ModernBERT's layer 0 has no attention norm
                order.append("")
                continue
            tensors[f"layer{layer}.{key}"] = np.ascontiguousarray(weights[name])
            order.append(f"layer{layer}.{key}")
    tensors["case.ids"] = new_ids.astype(np.int32)
    tensors["case.lengths"] = lengths.astype(np.int32)
    tensors["case.vectors"] = vectors.astype(np.float32)
    info = {
        "source": f"testdata/{bundle} (manifest.json, {art['files'][0]}, {m['reference']['file']})",
        "family": family, "architecture": arch, "embed": m["embed"], "order": order,
        "vocab_rows_kept": len(used), "word_rows": used,
    }
    save_file(tensors, os.path.join(HERE, out_name + ".safetensors"))
    with open(os.path.join(HERE, out_name + ".json"), "w") as f:
        json.dump(info, f, indent=1)
    print(out_name, len(used), "word rows,", sum(v.nbytes for v in tensors.values()), "bytes")


def quantize_golden():
    src = os.path.join(REF, "quantize", "sentence-transformers-145ef47d.txt")
    dst = os.path.join(HERE, "quantize-sentence-transformers-145ef47d.txt")
    with open(src, "rb") as f, open(dst, "wb") as g:
        g.write(f.read())


if __name__ == "__main__":
    if not os.path.isdir(REF):
        sys.exit("the reference's test data is not mounted here")
    one("tiny-bert-bundle", "tiny_bert")
    one("tiny-modernbert-bundle", "tiny_modernbert")
    one("tiny-nomic-bundle", "tiny_nomic")
    quantize_golden()
