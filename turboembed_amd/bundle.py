"""Model bundles: a directory with manifest.json, its weights and its
reference, read into the model description model_load takes.

As the reference core reads one:
- opening (core/src/bundle.rs:20-37): a directory with a manifest.json,
  else TURBO_E_BUNDLE_NOT_FOUND; a manifest that does not parse is
  TURBO_E_BUNDLE_INVALID;
- every file read is one the manifest lists, resolved inside the directory,
  of the listed size and SHA-256 (bundle.rs:39-125): else
  TURBO_E_BUNDLE_INVALID (unlisted, outside, not a regular file),
  TURBO_E_BUNDLE_NOT_FOUND (absent) or TURBO_E_BUNDLE_INTEGRITY (size or
  hash);
- the encoder's tensors are found by the artifact's tensor_names, `{layer}`
  replaced by the layer's index, in the family's TURBO_* order, each in
  exactly one of the artifact's safetensors files, all of one dtype (F32,
  F16 or BF16) (core/src/model/place.rs:132-200, model/mod.rs:230-330); a
  ModernBERT's layer 0 has no attention norm, its slot empty;
- the description's fields are the architecture's, rotary models adding
  the core's cos/sin table, their thetas (local defaults to global), the
  MLP, activation and norm kinds and the attention window
  (core/src/model/mod.rs:379-438, model/rotary.rs:121-155);
- a classifier (core/src/model/heads.rs:13-38) is a QA model's span head
  (handed to model_load) or a rerank model's pooler and classifier (applied
  on the host).

The rocm backend loads the BERT, RoBERTa, DeBERTa-v2, ModernBERT and
nomic-bert families from raw weights (FORMAT_SAFETENSORS); a bundle of another family
or format is TURBO_E_BUNDLE_NO_ARTIFACT here. Tokenizers are the caller's:
nothing here reads tokenizer.json.
"""
import hashlib
import json
import os
import struct

import numpy as np

from . import seam as S
from .model import ModelDesc

TURBO_E_BUNDLE_NOT_FOUND = 1280
TURBO_E_BUNDLE_INVALID = 1281
TURBO_E_BUNDLE_INTEGRITY = 1282
TURBO_E_BUNDLE_NO_ARTIFACT = 1283

FAMILIES = {"FAMILY_BERT": S.TURBO_FAMILY_BERT, "FAMILY_ROBERTA": S.TURBO_FAMILY_ROBERTA,
            "FAMILY_DEBERTA_V2": S.TURBO_FAMILY_DEBERTA_V2, "FAMILY_MODERNBERT": S.TURBO_FAMILY_MODERNBERT,
            "FAMILY_NOMIC_BERT": S.TURBO_FAMILY_NOMIC_BERT}

# The tensor roles of each family in TURBO_* order: embeddings, then a layer's
# (include/turbo/turbo_backend.h:63-153).
_BERT = (("word_embeddings", "position_embeddings", "token_type_embeddings", "embeddings_ln_weight",
          "embeddings_ln_bias"),
         ("q_weight", "q_bias", "k_weight", "k_bias", "v_weight", "v_bias", "attn_out_weight", "attn_out_bias",
          "attn_ln_weight", "attn_ln_bias", "ffn_in_weight", "ffn_in_bias", "ffn_out_weight", "ffn_out_bias",
          "ffn_ln_weight", "ffn_ln_bias"))
ROLES = {
    S.TURBO_FAMILY_BERT: _BERT,
    S.TURBO_FAMILY_ROBERTA: _BERT,
    S.TURBO_FAMILY_DEBERTA_V2: (("word_embeddings", "embeddings_ln_weight", "embeddings_ln_bias", "relative_embeddings",
                                 "relative_ln_weight", "relative_ln_bias"), _BERT[1]),
    S.TURBO_FAMILY_MODERNBERT: (("word_embeddings", "embeddings_ln_weight", "final_norm_weight"),
                                ("attn_ln_weight", "qkv_weight", "attn_out_weight", "ffn_ln_weight", "ffn_in_weight",
                                 "ffn_out_weight")),
    S.TURBO_FAMILY_NOMIC_BERT: (("word_embeddings", "token_type_embeddings", "embeddings_ln_weight",
                                 "embeddings_ln_bias"),
                                ("qkv_weight", "attn_out_weight", "attn_ln_weight", "attn_ln_bias", "ffn_gate_weight",
                                 "ffn_up_weight", "ffn_out_weight", "ffn_ln_weight", "ffn_ln_bias")),
}

# Weights are F32, F16 or BF16 (kept as its uint16 bits); a reference file
# also holds integer tensors (ids, lengths).
_ST_DTYPES = {"F32": np.float32, "F16": np.float16, "BF16": np.uint16, "F64": np.float64, "I64": np.int64,
              "I32": np.int32, "I16": np.int16, "I8": np.int8, "U8": np.uint8}
_WEIGHT_DTYPES = ("F32", "F16", "BF16")
_ENUMS = {
    "mlp": {"MLP_DENSE": S.TURBO_MLP_DENSE, "MLP_GATED": S.TURBO_MLP_GATED},
    "activation": {"ACTIVATION_GELU_ERF": S.TURBO_ACTIVATION_GELU_ERF, "ACTIVATION_SILU": S.TURBO_ACTIVATION_SILU},
    "norm": {"NORM_LAYER": S.TURBO_NORM_LAYER, "NORM_LAYER_NO_BIAS": S.TURBO_NORM_LAYER_NO_BIAS},
}
_POOLING = {"POOLING_MEAN": S.TURBO_POOLING_MEAN, "POOLING_CLS": S.TURBO_POOLING_CLS,
            "POOLING_LAST": S.TURBO_POOLING_LAST}
_NORMALIZE = {"NORMALIZE_NONE": S.TURBO_NORMALIZE_NONE, "NORMALIZE_L2": S.TURBO_NORMALIZE_L2}


def _error(code, message):
    from . import TurboError
    return TurboError(code, 0, message)


def parse_safetensors(name, data):
    """{tensor name: numpy array} of a safetensors file's bytes: an 8-byte
    little-endian header length, a JSON header of dtype, shape and
    data_offsets, then the data (BF16 as its uint16 bits)."""
    if len(data) < 8:
        raise _error(TURBO_E_BUNDLE_INVALID, f"{name}: {len(data)} bytes is no safetensors file")
    n = struct.unpack_from("<Q", data, 0)[0]
    if 8 + n > len(data):
        raise _error(TURBO_E_BUNDLE_INVALID, f"{name}: a header of {n} bytes in a file of {len(data)}")
    try:
        header = json.loads(bytes(data[8:8 + n]))
    except ValueError as e:
        raise _error(TURBO_E_BUNDLE_INVALID, f"{name}: header: {e}") from None
    body = memoryview(data)[8 + n:]
    out = {}
    for k, v in header.items():
        if k == "__metadata__":
            continue
        dt = v.get("dtype")
        shape = tuple(int(x) for x in v.get("shape", ()))
        lo, hi = (int(x) for x in v.get("data_offsets", (0, 0)))
        if dt not in _ST_DTYPES:
            out[k] = (dt, shape, None)
            continue
        np_dt = np.dtype(_ST_DTYPES[dt]).newbyteorder("<")
        if not 0 <= lo <= hi <= len(body) or hi - lo != int(np.prod(shape, dtype=np.int64)) * np_dt.itemsize:
            raise _error(TURBO_E_BUNDLE_INVALID, f"{name}: {k}: offsets {lo}..{hi} do not hold {dt}{list(shape)}")
        out[k] = (dt, shape, np.frombuffer(body[lo:hi], dtype=np_dt).reshape(shape))
    return out


class Bundle:
    """An opened bundle directory."""

    def __init__(self, path):
        if not os.path.isdir(path):
            raise _error(TURBO_E_BUNDLE_NOT_FOUND, f"{path} is not a directory")
        self.dir = os.path.realpath(path)
        mf = os.path.join(self.dir, "manifest.json")
        if not os.path.isfile(mf):
            raise _error(TURBO_E_BUNDLE_NOT_FOUND, f"{path}: no manifest.json")
        raw = open(mf, "rb").read()
        try:
            self.manifest = json.loads(raw)
        except ValueError as e:
            raise _error(TURBO_E_BUNDLE_INVALID, f"manifest.json: {e}") from None
        self.manifest_sha256 = hashlib.sha256(raw).hexdigest()
        self.files = {f["path"]: f for f in self.manifest.get("files", [])}
        self.task = self.manifest.get("task", "TASK_EMBED")

    # -- files ------------------------------------------------------------------
    def read_verified(self, rel):
        """The bytes of a listed file, checked against its size and hash."""
        entry = self.files.get(rel)
        if entry is None:
            raise _error(TURBO_E_BUNDLE_INVALID, f"{rel}: not among the manifest's files")
        joined = os.path.join(self.dir, rel)
        if not os.path.lexists(joined):
            raise _error(TURBO_E_BUNDLE_NOT_FOUND, f"{rel} is absent")
        real = os.path.realpath(joined)
        if not os.path.exists(real):
            raise _error(TURBO_E_BUNDLE_INVALID, f"{rel}: a link to nothing")
        if os.path.commonpath([real, self.dir]) != self.dir:
            raise _error(TURBO_E_BUNDLE_INVALID, f"{rel} resolves outside the bundle directory")
        if not os.path.isfile(real):
            raise _error(TURBO_E_BUNDLE_INVALID, f"{rel} is not a regular file")
        data = open(real, "rb").read()
        if len(data) != int(entry["size"]):
            raise _error(TURBO_E_BUNDLE_INTEGRITY, f"{rel}: size is {len(data)}, the manifest says {entry['size']}")
        h = hashlib.sha256(data).hexdigest()
        if h != entry["sha256"]:
            raise _error(TURBO_E_BUNDLE_INTEGRITY, f"{rel}: SHA-256 is {h}, the manifest says {entry['sha256']}")
        return data

    def _tensors(self, art):
        files = [(f, parse_safetensors(f, self.read_verified(f))) for f in art["files"]]

        def find(name, what):
            hits = [(f, t[name]) for f, t in files if name in t]
            if not hits:
                raise _error(TURBO_E_BUNDLE_INVALID, f"{', '.join(art['files'])}: no tensor {name!r} ({what})")
            if len(hits) > 1:
                raise _error(TURBO_E_BUNDLE_INVALID, f"{name!r} ({what}) is in both {hits[0][0]} and {hits[1][0]}")
            f, (dt, shape, arr) = hits[0]
            if dt not in _WEIGHT_DTYPES:
                raise _error(TURBO_E_BUNDLE_INVALID, f"{f}: {name} ({what}) is {dt}; weights are F32, F16 or BF16")
            return dt, arr
        return find

    # -- the model --------------------------------------------------------------
    @property
    def architecture(self):
        a = self.manifest.get("architecture")
        if a is None:
            raise _error(TURBO_E_BUNDLE_NO_ARTIFACT, "the bundle has no architecture (a static or compiled model)")
        return a

    def model_desc(self, artifact=0):
        """The ModelDesc of the artifact: the encoder's tensors in TURBO_*
        order, the rotary fields, and a QA model's span head."""
        a = self.architecture
        family = FAMILIES.get(a.get("family"))
        if family is None:
            raise _error(TURBO_E_BUNDLE_NO_ARTIFACT, f"family {a.get('family')}: the rocm backend loads BERT, "
                                                     "RoBERTa, DeBERTa-v2, ModernBERT and nomic-bert encoders")
        arts = self.manifest.get("artifacts", [])
        if not 0 <= artifact < len(arts):
            raise _error(S.TURBO_E_INVALID_ARGUMENT, f"artifact {artifact}: bundle has {len(arts)} artifacts")
        art = arts[artifact]
        if art.get("format", "FORMAT_SAFETENSORS") != "FORMAT_SAFETENSORS":
            raise _error(TURBO_E_BUNDLE_NO_ARTIFACT, f"artifact {art.get('name')}: {art.get('format')} (the rocm "
                                                     "backend loads raw weights)")
        names = art.get("tensor_names", {})
        find = self._tensors(art)
        emb, per = ROLES[family]
        tensors, labels, dtype = [], [], None

        def take(role, layer=None):
            nonlocal dtype
            name = names.get(role)
            if name is None:
                raise _error(TURBO_E_BUNDLE_INVALID, f"artifacts[{artifact}].tensor_names: no {role}")
            if layer is not None:
                name = name.replace("{layer}", str(layer))
            dt, arr = find(name, role)
            if dtype is None:
                dtype = dt
            elif dt != dtype:
                raise _error(TURBO_E_BUNDLE_INVALID, f"{name} ({role}) is {dt}; the other weights are {dtype}")
            tensors.append(arr)
            labels.append(name)

        for role in emb:
            take(role)
        for layer in range(int(a["layers"])):
            for role in per:
                if family == S.TURBO_FAMILY_MODERNBERT and layer == 0 and role == "attn_ln_weight":
                    tensors.append(None)      # layer 0 reads the embeddings' rows as they are
                    labels.append("absent")
                    continue
                take(role, layer)
        kw = {}
        if family in (S.TURBO_FAMILY_MODERNBERT, S.TURBO_FAMILY_NOMIC_BERT):
            rope = a.get("rope") or {}
            if "global_theta" not in rope:
                raise _error(TURBO_E_BUNDLE_INVALID, "architecture.rope: a rotary family needs global_theta")
            g = float(rope["global_theta"])
            att = a.get("attention") or {}
            kw = dict(rope=(g, float(rope.get("local_theta", g))), attention_window=int(att.get("window", 0)),
                      global_every=int(att.get("global_every", 0)),
                      mlp=_ENUMS["mlp"][a.get("mlp", "MLP_DENSE")],
                      activation=_ENUMS["activation"][a.get("activation", "ACTIVATION_GELU_ERF")],
                      norm=_ENUMS["norm"][a.get("norm", "NORM_LAYER")])
        if family == S.TURBO_FAMILY_DEBERTA_V2:
            rel = a.get("relative") or {}
            if "position_buckets" not in rel or "max_relative_positions" not in rel:
                raise _error(TURBO_E_BUNDLE_INVALID, "architecture.relative: a DeBERTa-v2 model needs position_buckets "
                                                     "and max_relative_positions")
            kw["relative"] = (int(rel["position_buckets"]), int(rel["max_relative_positions"]))
        c = self.manifest.get("classifier")
        if self.task == "TASK_EXTRACTIVE_QA" and c is not None:
            kw["span_head"] = self._classifier(find, names, a, c)[2:]
        return ModelDesc(family, int(a["layers"]), int(a["hidden"]), int(a["heads"]), int(a["intermediate"]),
                         int(a["vocab_size"]), int(a["max_positions"]), int(a.get("token_types", 0)),
                         float(a["layer_norm_eps"]), tensors, position_offset=int(a.get("position_offset", 0)),
                         names=labels, **kw)

    @staticmethod
    def _classifier(find, names, a, c):
        """(pooler weight, pooler bias, classifier weight, classifier bias) as F32, the pooler's None when absent."""
        h, n = int(a["hidden"]), len(c.get("labels", []))
        pw, pb = names.get("pooler_weight"), names.get("pooler_bias")
        if (pw is None) != (pb is None):
            raise _error(TURBO_E_BUNDLE_INVALID, "tensor_names: pooler_weight and pooler_bias come together, or neither")

        def f32(name, role, shape):
            if name is None:
                raise _error(TURBO_E_BUNDLE_INVALID, f"tensor_names: no {role}, which a classifier needs")
            dt, arr = find(name, role)
            if arr.shape != shape:
                raise _error(TURBO_E_BUNDLE_INVALID, f"{name} ({role}) is {list(arr.shape)}, not {list(shape)}")
            if dt == "BF16":
                return (arr.astype(np.uint32) << 16).view(np.float32)
            return arr.astype(np.float32)
        pooler = (f32(pw, "pooler_weight", (h, h)), f32(pb, "pooler_bias", (h,))) if pw else (None, None)
        return pooler + (f32(names.get("classifier_weight"), "classifier_weight", (n, h)),
                         f32(names.get("classifier_bias"), "classifier_bias", (n,)))

    def rerank_head(self, artifact=0):
        """A rerank model's head as rerank.RerankHead's keywords: pooler
        (when the bundle has one) and the one-label classifier."""
        c = self.manifest.get("classifier")
        if self.task != "TASK_RERANK" or c is None:
            raise _error(S.TURBO_E_UNSUPPORTED_TASK, "the bundle is not a rerank model")
        art = self.manifest["artifacts"][artifact]
        pw, pb, cw, cb = self._classifier(self._tensors(art), art.get("tensor_names", {}), self.architecture, c)
        return dict(classifier_weight=cw, classifier_bias=float(cb[0]), pooler_weight=pw, pooler_bias=pb)

    # -- what the bundle says of runs ----------------------------------------------
    def embed_defaults(self):
        """(pooling, normalize, dim, max_seq, max_batch) of the manifest's embed block."""
        e = self.manifest.get("embed") or {}
        return (_POOLING.get(e.get("pooling"), S.TURBO_POOLING_MEAN),
                _NORMALIZE.get(e.get("normalize"), S.TURBO_NORMALIZE_NONE), int(e.get("dim", 0)),
                int(e.get("max_seq", 0)), int(e.get("max_batch", 0)))

    def reference(self):
        """The sealed reference file's tensors (e.g. ids, lengths and the
        upstream vectors), verified like every other file."""
        ref = self.manifest.get("reference") or {}
        if "file" not in ref:
            raise _error(TURBO_E_BUNDLE_INVALID, "the manifest names no reference file")
        t = parse_safetensors(ref["file"], self.read_verified(ref["file"]))
        return {k: v[2] for k, v in t.items() if v[2] is not None}
