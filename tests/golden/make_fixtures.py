"""Writes the golden fixtures under tests/golden/ from the reference's test data.

Run here, where the reference tree is mounted; the fixtures it writes are
committed, and nothing at test time reads the reference.

For each sealed tiny bundle (testdata/tiny-bert-bundle, tiny-modernbert-bundle, tiny-deberta-bundle,
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


def deberta_order():
    return (["word_embeddings", "embeddings_ln_weight", "embeddings_ln_bias", "relative_embeddings", "relative_ln_weight",
             "relative_ln_bias"], bert_order(0)[1])


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
                "FAMILY_NOMIC_BERT": nomic_order(), "FAMILY_DEBERTA_V2": deberta_order()}[family]
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


def rerank_fixture():
    """tiny_rerank: testdata/tiny-rerank-reference's transformers scores for
    four (query, passage) pairs over the tiny BERT encoder, with its pooler
    and classifier (head.safetensors), the encoder's weights (word rows
    reduced as above), and each pair's query and passage token ids.

    The reference holds each pair's first window (ids, types, length) and
    its max-over-windows score. Query and passage ids are read from that
    window ([CLS] query [SEP] passage [SEP], types 1 from the passage on);
    the one pair whose window is full (length 32 = max_tokens) repeats one
    word in both texts (cases.json), so its query and passage are that
    word's one token id repeated as many times as the text has words."""
    d = os.path.join(REF, "tiny-rerank-reference")
    ref = load_file(os.path.join(d, "reference.safetensors"))
    head = load_file(os.path.join(d, "head.safetensors"))
    cases = json.load(open(os.path.join(d, "cases.json")))
    bundle = os.path.join(REF, "tiny-bert-bundle")
    m = json.load(open(os.path.join(bundle, "manifest.json")))
    arch = m["architecture"]
    art = m["artifacts"][0]
    names = art["tensor_names"]
    weights = load_file(os.path.join(bundle, art["files"][0]))
    max_tokens, query_tokens = 32, 8
    queries, passages = [], []
    for i, case in enumerate(cases):
        n = int(ref["lengths"][i])
        row, ty = ref["ids"][i, :n], ref["types"][i, :n]
        b = int(np.argmax(ty == 1))
        q, p = [int(v) for v in row[1:b - 1]], [int(v) for v in row[b:n - 1]]
        if n == max_tokens:
            qw, pw = case["text"].split(), case["passage"].split()
            assert len(set(qw)) == 1 and len(set(pw)) == 1 and len(set(q)) == 1 and len(set(p)) == 1
            q, p = q[:1] * len(qw), p[:1] * len(pw)
        queries.append(q)
        passages.append(p)
    used = sorted({0, 101, 102} | {v for q in queries for v in q} | {v for p in passages for v in p})
    remap = {old: new for new, old in enumerate(used)}
    emb, per = bert_order(arch["layers"])
    tensors, order = {}, []
    for key in emb:
        t = weights[names[key]]
        if key == "word_embeddings":
            t = t[used]
        tensors[f"emb.{key}"] = np.ascontiguousarray(t)
        order.append(f"emb.{key}")
    for layer in range(arch["layers"]):
        for key in per:
            name = names[key].replace("{layer}", str(layer))
            tensors[f"layer{layer}.{key}"] = np.ascontiguousarray(weights[name])
            order.append(f"layer{layer}.{key}")
    for k in ("bert.pooler.dense.weight", "bert.pooler.dense.bias", "classifier.weight", "classifier.bias"):
        tensors["head." + k] = np.ascontiguousarray(head[k])
    first = np.vectorize(lambda v: remap[int(v)] if int(v) in remap else 0)(ref["ids"]).astype(np.int32)
    tensors["case.first_ids"] = first
    tensors["case.first_types"] = ref["types"].astype(np.int32)
    tensors["case.first_lengths"] = ref["lengths"].astype(np.int32)
    tensors["case.scores"] = ref["scores"].astype(np.float32).ravel()
    info = {
        "source": "testdata/tiny-rerank-reference (reference.safetensors, head.safetensors, cases.json) over "
                  "testdata/tiny-bert-bundle (manifest.json, weights)",
        "family": arch["family"], "architecture": arch, "order": order, "vocab_rows_kept": len(used),
        "word_rows": used, "start_id": remap[101], "end_id": remap[102], "pad_id": 0,
        "max_tokens": max_tokens, "query_tokens": query_tokens, "max_batch": 4, "template": "PAIR_BERT",
        "queries": [[remap[v] for v in q] for q in queries],
        "passages": [[remap[v] for v in p] for p in passages],
    }
    save_file(tensors, os.path.join(HERE, "tiny_rerank.safetensors"))
    with open(os.path.join(HERE, "tiny_rerank.json"), "w") as f:
        json.dump(info, f, indent=1)
    print("tiny_rerank", len(used), "word rows")


def qa_fixture():
    """tiny_qa: testdata/tiny-qa-reference's transformers start and end
    logits for every token of six QA windows over the tiny BERT encoder,
    with its span head (head.safetensors: qa_outputs, [2, hidden] and [2]),
    the encoder's weights (word rows reduced as above) and the windows'
    ids, types and lengths as the reference holds them. Logits are [105, 2]:
    the windows' live tokens in order, start then end."""
    d = os.path.join(REF, "tiny-qa-reference")
    ref = load_file(os.path.join(d, "reference.safetensors"))
    head = load_file(os.path.join(d, "head.safetensors"))
    cases = json.load(open(os.path.join(d, "cases.json")))
    bundle = os.path.join(REF, "tiny-bert-bundle")
    m = json.load(open(os.path.join(bundle, "manifest.json")))
    arch = m["architecture"]
    names = m["artifacts"][0]["tensor_names"]
    weights = load_file(os.path.join(bundle, m["artifacts"][0]["files"][0]))
    ids, lengths = ref["ids"], ref["lengths"]
    used = sorted({0} | {int(v) for r, n in zip(ids, lengths) for v in r[:n]})
    remap = {old: new for new, old in enumerate(used)}
    new_ids = np.zeros_like(ids)
    for i, (r, n) in enumerate(zip(ids, lengths)):
        new_ids[i, :n] = [remap[int(v)] for v in r[:n]]
    emb, per = bert_order(arch["layers"])
    tensors, order = {}, []
    for key in emb:
        t = weights[names[key]]
        if key == "word_embeddings":
            t = t[used]
        tensors[f"emb.{key}"] = np.ascontiguousarray(t)
        order.append(f"emb.{key}")
    for layer in range(arch["layers"]):
        for key in per:
            name = names[key].replace("{layer}", str(layer))
            tensors[f"layer{layer}.{key}"] = np.ascontiguousarray(weights[name])
            order.append(f"layer{layer}.{key}")
    tensors["head.weight"] = np.ascontiguousarray(head["qa_outputs.weight"], np.float32)
    tensors["head.bias"] = np.ascontiguousarray(head["qa_outputs.bias"], np.float32)
    tensors["case.ids"] = new_ids.astype(np.int32)
    tensors["case.types"] = ref["types"].astype(np.int32)
    tensors["case.lengths"] = lengths.astype(np.int32)
    tensors["case.logits"] = ref["logits"].astype(np.float32)
    info = {
        "source": "testdata/tiny-qa-reference (reference.safetensors, head.safetensors, cases.json) over "
                  "testdata/tiny-bert-bundle (manifest.json, weights)",
        "family": arch["family"], "architecture": arch, "order": order, "vocab_rows_kept": len(used),
        "word_rows": used, "pad_id": 0, "qa": cases["qa"],
    }
    save_file(tensors, os.path.join(HERE, "tiny_qa.safetensors"))
    with open(os.path.join(HERE, "tiny_qa.json"), "w") as f:
        json.dump(info, f, indent=1)
    print("tiny_qa", len(used), "word rows")


def bundle_files():
    """tiny-modernbert-bundle as it is sealed (manifest.json, its weights and
    its reference; the tokenizer is not read here and stays out), and the
    manifests of tiny-bert-bundle and tiny-nomic-bundle, whose tensor names
    the bundle tests build weights files under."""
    src = os.path.join(REF, "tiny-modernbert-bundle")
    dst = os.path.join(HERE, "tiny-modernbert-bundle")
    for rel in ("manifest.json", "weights/model.safetensors", "reference/reference.safetensors"):
        os.makedirs(os.path.dirname(os.path.join(dst, rel)), exist_ok=True)
        with open(os.path.join(src, rel), "rb") as f, open(os.path.join(dst, rel), "wb") as g:
            g.write(f.read())
    os.makedirs(os.path.join(HERE, "manifests"), exist_ok=True)
    for b in ("tiny-bert-bundle", "tiny-nomic-bundle"):
        with open(os.path.join(REF, b, "manifest.json"), "rb") as f, \
                open(os.path.join(HERE, "manifests", b + ".json"), "wb") as g:
            g.write(f.read())


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
    one("tiny-deberta-bundle", "tiny_deberta")
    rerank_fixture()
    qa_fixture()
    bundle_files()
    quantize_golden()
