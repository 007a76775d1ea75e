"""Bundles read into model descriptions (turboembed_amd/bundle.py), on the CPU.

The sealed tiny ModernBERT bundle is read as it is sealed (its files'
hashes checked) and its description, through the oracle, meets the upstream
vectors the bundle holds. The tiny BERT and nomic bundles are rebuilt under
their real manifests' tensor names from the golden fixtures' tensors (each
placed by its role's name, the word table cut to the rows the cases use),
so a wrong role order or name in the reader breaks their vectors. The QA
and rerank bundles are the tiny BERT under those tasks, as the reference's
own tests make them (core/tests/qa/common.rs:17-50). The refusals are
bundle.rs's.
"""
import copy
import hashlib
import json
import os
import shutil

import numpy as np
import pytest
from safetensors.numpy import save_file

import oracle
import turboembed_amd as T
from turboembed_amd import bundle as B
from turboembed_amd import seam as S

import small

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SEALED = os.path.join(GOLDEN, "tiny-modernbert-bundle")


def _close(got, want):
    assert small.cosine_rows(got, want).min() >= 0.9999
    assert np.abs(got - want).max() <= 1e-4


def _vectors(desc, bundle):
    ref = bundle.reference()
    ids = ref["ids"].astype(np.int32)
    mask = (np.arange(ids.shape[1])[None, :] < ref["lengths"][:, None]).astype(np.int32)
    pooling, normalize, dim, _, _ = bundle.embed_defaults()
    return oracle.encode(desc, ids, mask, pooling=pooling, normalize=normalize, output_dim=dim), ref


def test_the_sealed_modernbert_bundle_meets_its_upstream_vectors():
    b = B.Bundle(SEALED)
    desc = b.model_desc()
    assert desc.family == S.TURBO_FAMILY_MODERNBERT and desc.layers == 3 and desc.tensors[3] is None
    assert desc.rope == (160000.0, 10000.0) and (desc.attention_window, desc.global_every) == (8, 3)
    assert (desc.mlp, desc.norm) == (S.TURBO_MLP_GATED, S.TURBO_NORM_LAYER_NO_BIAS)
    got, ref = _vectors(desc, b)
    _close(got, ref["embeddings"])
    # The same tensors as the golden fixture's, its word table cut to the rows it keeps.
    fdesc, _, _, _, info = oracle.fixture("tiny_modernbert")
    assert np.array_equal(desc.tensors[0][info["word_rows"]], fdesc.tensors[0])
    for a, f in zip(desc.tensors[1:], fdesc.tensors[1:]):
        assert (a is None and f is None) or np.array_equal(a, f)


def _write_bundle(dir, manifest, weights, reference):
    os.makedirs(os.path.join(dir, "weights"), exist_ok=True)
    os.makedirs(os.path.join(dir, "reference"), exist_ok=True)
    save_file(weights, os.path.join(dir, "weights", "model.safetensors"))
    save_file(reference, os.path.join(dir, "reference", "reference.safetensors"))
    files = []
    for rel in ("weights/model.safetensors", "reference/reference.safetensors"):
        data = open(os.path.join(dir, rel), "rb").read()
        files.append({"path": rel, "size": len(data), "sha256": hashlib.sha256(data).hexdigest()})
    manifest = copy.deepcopy(manifest)
    manifest["files"] = files
    manifest["artifacts"][0]["files"] = ["weights/model.safetensors"]
    manifest["reference"]["file"] = "reference/reference.safetensors"
    with open(os.path.join(dir, "manifest.json"), "w") as f:
        json.dump(manifest, f)
    return dir


def _rebuilt(tmp_path, fixture, manifest_name, extra=None, task=None):
    """A bundle of the golden fixture's tensors under the real manifest's names."""
    from safetensors.numpy import load_file
    t = load_file(os.path.join(GOLDEN, fixture + ".safetensors"))
    info = json.load(open(os.path.join(GOLDEN, fixture + ".json")))
    m = json.load(open(os.path.join(GOLDEN, "manifests", manifest_name + ".json")))
    names = m["artifacts"][0]["tensor_names"]
    weights = {}
    for key in info["order"]:
        if not key:
            continue
        part, role = key.split(".", 1)
        layer = None if part == "emb" else part[len("layer"):]
        weights[names[role].replace("{layer}", layer) if layer is not None else names[role]] = t[key]
    m["architecture"]["vocab_size"] = info["vocab_rows_kept"]
    if extra:
        for k, v in extra(t).items():
            weights[k] = v
    ref = {k.split(".", 1)[1]: v for k, v in t.items() if k.startswith("case.")}
    ref = {"ids": ref.get("ids", ref.get("first_ids")), "lengths": ref.get("lengths", ref.get("first_lengths")),
           "embeddings": ref.get("vectors", np.zeros((1, 1), np.float32))}
    if task:
        task(m)
    return B.Bundle(_write_bundle(str(tmp_path / manifest_name), m, weights, ref))


@pytest.mark.parametrize("fixture,manifest", [("tiny_bert", "tiny-bert-bundle"), ("tiny_nomic", "tiny-nomic-bundle")])
def test_bundles_under_their_real_tensor_names_meet_the_upstream_vectors(tmp_path, fixture, manifest):
    b = _rebuilt(tmp_path, fixture, manifest)
    got, ref = _vectors(b.model_desc(), b)
    _close(got, ref["embeddings"])


def test_a_qa_bundle_carries_its_span_head(tmp_path):
    def qa(m):
        m.pop("embed", None)
        m["task"] = "TASK_EXTRACTIVE_QA"
        m["classifier"] = {"kind": "CLASSIFIER_TOKEN", "labels": ["start", "end"]}
        m["artifacts"][0]["tensor_names"]["classifier_weight"] = "qa_outputs.weight"
        m["artifacts"][0]["tensor_names"]["classifier_bias"] = "qa_outputs.bias"
    b = _rebuilt(tmp_path, "tiny_qa", "tiny-bert-bundle", task=qa,
                 extra=lambda t: {"qa_outputs.weight": t["head.weight"], "qa_outputs.bias": t["head.bias"]})
    desc = b.model_desc()
    qd, windows, logits, info = oracle.qa_fixture()
    assert np.array_equal(desc.span_head[0], qd.span_head[0]) and np.array_equal(desc.span_head[1], qd.span_head[1])
    got = oracle.qa_logits(desc, windows, info["pad_id"])
    assert np.abs(got - logits).max() <= 1e-4 * np.abs(logits).max()


def test_a_rerank_bundle_carries_its_pooler_and_classifier(tmp_path):
    def rr(m):
        m.pop("embed", None)
        m["task"] = "TASK_RERANK"
        m["classifier"] = {"kind": "CLASSIFIER_SEQUENCE", "labels": ["score"]}
        tn = m["artifacts"][0]["tensor_names"]
        tn.update(pooler_weight="bert.pooler.dense.weight", pooler_bias="bert.pooler.dense.bias",
                  classifier_weight="classifier.weight", classifier_bias="classifier.bias")
    b = _rebuilt(tmp_path, "tiny_rerank", "tiny-bert-bundle", task=rr,
                 extra=lambda t: {k[len("head."):]: v for k, v in t.items() if k.startswith("head.")})
    desc, pairs, head, info, ref = oracle.rerank_fixture()
    got = b.rerank_head()
    for k in ("classifier_weight", "pooler_weight", "pooler_bias"):
        assert np.array_equal(np.ravel(got[k]), np.ravel(head[k])), k
    assert got["classifier_bias"] == head["classifier_bias"]
    scores = oracle.rerank(b.model_desc(), pairs, got, info["start_id"], info["end_id"],
                           query_tokens=info["query_tokens"], max_tokens=info["max_tokens"])
    assert np.abs(scores - ref["scores"]).max() <= 1e-4 * np.abs(ref["scores"]).max()


def _code(fn):
    with pytest.raises(T.TurboError) as e:
        fn()
    return e.value.code


def test_a_bundle_is_refused_as_the_core_refuses_it(tmp_path):
    d = str(tmp_path / "b")
    shutil.copytree(SEALED, d)
    w = os.path.join(d, "weights", "model.safetensors")
    good = open(w, "rb").read()
    assert _code(lambda: B.Bundle(str(tmp_path / "none"))) == B.TURBO_E_BUNDLE_NOT_FOUND
    # A changed byte, then a changed size.
    bad = bytearray(good)
    bad[-1] ^= 1
    open(w, "wb").write(bytes(bad))
    assert _code(lambda: B.Bundle(d).model_desc()) == B.TURBO_E_BUNDLE_INTEGRITY
    open(w, "wb").write(good + b"\0")
    assert _code(lambda: B.Bundle(d).model_desc()) == B.TURBO_E_BUNDLE_INTEGRITY
    open(w, "wb").write(good)
    B.Bundle(d).model_desc()
    # A file the manifest does not list; one it lists that is absent; one
    # that resolves outside the bundle.
    b = B.Bundle(d)
    assert _code(lambda: b.read_verified("weights/other.safetensors")) == B.TURBO_E_BUNDLE_INVALID
    os.remove(os.path.join(d, "reference", "reference.safetensors"))
    assert _code(lambda: b.reference()) == B.TURBO_E_BUNDLE_NOT_FOUND
    outside = str(tmp_path / "outside.safetensors")
    shutil.copy(os.path.join(SEALED, "reference", "reference.safetensors"), outside)
    os.symlink(outside, os.path.join(d, "reference", "reference.safetensors"))
    assert _code(lambda: b.reference()) == B.TURBO_E_BUNDLE_INVALID
    # A family the backend does not load, and a manifest that does not parse.
    m = json.load(open(os.path.join(d, "manifest.json")))
    m["architecture"]["family"] = "FAMILY_STATIC"
    json.dump(m, open(os.path.join(d, "manifest.json"), "w"))
    assert _code(lambda: B.Bundle(d).model_desc()) == B.TURBO_E_BUNDLE_NO_ARTIFACT
    open(os.path.join(d, "manifest.json"), "w").write("{")
    assert _code(lambda: B.Bundle(d)) == B.TURBO_E_BUNDLE_INVALID
