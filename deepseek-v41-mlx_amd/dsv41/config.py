"""Configuration of the attention path: the reference's ``ModelArgs``
(deepseek_v41_mlx/config.py:28-106), loaded from either release layout.

Design:

* ``_KEYS`` is one table, ``(attribute, JSON names tried in order, default)``, holding every
  attribute the reference defines (config.py:30-102) with its default and the JSON names its
  ``from_dict`` reads (config.py:146-191). The first JSON name that is present and not null
  wins. The same table serves keyword construction, the flat inference ``config.json`` and the
  HF hub file (whose ``text_config`` is folded over its top level first, config.py:137-140).
  YaRN settings may also arrive inside a ``rope_scaling`` object (config.py:142, 179-183);
  ``_ROPE_SCALING`` names them. Two fields differ between the two routes, as in the reference:
  a file without ``swiglu_limit`` gives 0.0 (the keyword default is 10.0), and a file never
  sets ``vision_n_layers`` (text-only runtime).
* Only the attention path's fields are read here. The MoE, hyper-connection, engram and
  side-path fields are pass-through entries: they carry the reference's names, defaults and
  JSON aliases so model code that reads e.g. ``args.hc_mult`` or ``args.n_activated_experts``
  runs, but nothing here interprets them. Keys outside the table (vision sizes, tokenizer ids
  ...) are kept verbatim in ``extra`` and reachable as attributes.
* The sharing topology is resolved by one walk down the layer stack
  (``_resolve_sources``): a compressing layer reads the latest KV source at or above it,
  whose compress ratio must equal its own, and the latest index source at or above it.
  This is the rule of config.py:108-133, evaluated for all layers at once; lookups raise
  ``ValueError`` for a layer the walk could not resolve.
"""

from __future__ import annotations

_TUPLE = tuple

# attribute, JSON names (flat layout name last unless they coincide), default
_KEYS = (
    ("dim", ("hidden_size", "dim"), 5120),
    ("n_layers", ("num_hidden_layers", "n_layers"), 40),
    ("n_heads", ("num_attention_heads", "n_heads"), 64),
    ("head_dim", ("head_dim",), 512),
    ("rope_head_dim", ("qk_rope_head_dim", "rope_head_dim"), 64),
    ("q_lora_rank", ("q_lora_rank",), 1280),
    ("o_lora_rank", ("o_lora_rank",), 1024),
    ("o_groups", ("o_groups",), 8),
    ("window_size", ("sliding_window", "window_size"), 128),
    ("norm_eps", ("rms_norm_eps", "norm_eps"), 1e-20),
    ("compress_ratios", ("compress_ratios",), ()),
    ("kv_source_layers", ("kv_source_layer_ids", "kv_source_layers"), ()),
    ("index_source_layers", ("index_source_layer_ids", "index_source_layers"), ()),
    ("compress_rope_theta", ("compress_rope_theta",), 160000.0),
    ("candidate_source_layer", ("candidate_source_layer_id", "candidate_source_layer"), -1),
    ("candidate_topk_blocks", ("candidate_topk_blocks",), 0),
    ("candidate_block_size", ("candidate_block_size",), 0),
    ("original_seq_len", ("original_seq_len",), 65536),
    ("rope_theta", ("rope_theta",), 10000.0),
    ("rope_factor", ("rope_factor",), 16.0),
    ("beta_fast", ("beta_fast",), 32),
    ("beta_slow", ("beta_slow",), 1),
    ("max_seq_len", ("max_position_embeddings", "max_seq_len"), 1048576),
    ("index_n_heads", ("index_n_heads",), 32),
    ("index_head_dim", ("index_head_dim",), 128),
    ("index_topk", ("index_topk",), 512),
    # pass-through: read by model code outside the attention path, never interpreted here
    ("vocab_size", ("vocab_size",), 129280),
    ("moe_inter_dim", ("moe_intermediate_size", "moe_inter_dim"), 2304),
    ("n_routed_experts", ("n_routed_experts",), 384),
    ("n_shared_experts", ("n_shared_experts",), 1),
    ("n_activated_experts", ("num_experts_per_tok", "n_activated_experts"), 6),
    ("score_func", ("scoring_func", "score_func"), "sqrtsoftplus"),
    ("gate_temp", ("gate_temp",), 1.0),
    ("norm_topk_prob", ("norm_topk_prob",), True),
    ("route_scale", ("routed_scaling_factor", "route_scale"), 1.5),
    ("swiglu_limit", ("swiglu_limit",), 10.0),
    ("hc_mult", ("hc_mult",), 4),
    ("hc_sinkhorn_iters", ("hc_sinkhorn_iters",), 20),
    ("hc_eps", ("hc_eps",), 1e-6),
    ("engram_layer_ids", ("engram_layer_ids",), ()),
    ("engram_num_embeddings", ("engram_num_embeddings",), ()),
    ("engram_max_ngram_size", ("engram_max_ngram_size",), 4),
    ("engram_vocab_size", ("engram_vocab_size",), 0),
    ("engram_n_heads", ("engram_n_heads",), 0),
    ("engram_head_dim", ("engram_head_dim",), 0),
    ("engram_pad_id", ("engram_pad_token_id", "engram_pad_id"), 2),
    ("engram_compressed_vocab_size", ("engram_compressed_vocab_size",), 0),
    ("n_mtp_layers", ("num_nextn_predict_layers", "n_mtp_layers"), 0),
    ("dspark_target_layer_ids", ("dspark_target_layer_ids",), ()),
    ("vision_n_layers", ("vision_n_layers",), 0),
)

# a release file that omits these gets a different value than keyword construction
# (config.py:162, 193): the file route's default, and a field the file route never sets
_FILE_DEFAULTS = {"swiglu_limit": 0.0}
_FILE_FIXED = {"vision_n_layers": 0}

# attribute -> its name inside a ``rope_scaling`` object, which takes precedence
_ROPE_SCALING = {"original_seq_len": "original_max_position_embeddings",
                 "rope_factor": "factor", "beta_fast": "beta_fast", "beta_slow": "beta_slow"}

_SEQUENCE_FIELDS = {"compress_ratios", "kv_source_layers", "index_source_layers"}
_TUPLE_FIELDS = {"engram_layer_ids", "engram_num_embeddings", "dspark_target_layer_ids"}
_FIELDS = {name for name, _, _ in _KEYS}


def _first(d: dict, names):
    for n in names:
        v = d.get(n)
        if v is not None:
            return v
    return None


class ModelArgs:
    """Attention-path configuration; attribute names and defaults are the reference's."""

    def __init__(self, **kw):
        extra = {k: kw.pop(k) for k in list(kw) if k not in _FIELDS}
        for name, _, default in _KEYS:
            v = kw.get(name, default)
            if name in _SEQUENCE_FIELDS:
                v = _TUPLE(int(x) for x in (v or ()))
            elif name in _TUPLE_FIELDS:
                v = _TUPLE(v or ())
            setattr(self, name, v)
        # not typed attributes of this path; kept so a release config round-trips
        self.extra = extra
        self._sources = None

    def __getattr__(self, name):
        # only reached for names that are not regular attributes
        extra = self.__dict__.get("extra", {})
        if name in extra:
            return extra[name]
        raise AttributeError(f"ModelArgs has no field {name!r}")

    def __repr__(self) -> str:
        body = ", ".join(f"{n}={getattr(self, n)!r}" for n, _, _ in _KEYS)
        return f"ModelArgs({body})"

    def __eq__(self, other) -> bool:
        return (isinstance(other, ModelArgs)
                and all(getattr(self, n) == getattr(other, n) for n in _FIELDS)
                and self.extra == other.extra)

    # ---------------------------------------------------------------- derived sizes

    @property
    def nope_head_dim(self) -> int:
        return self.head_dim - self.rope_head_dim

    def compress_ratio(self, layer_id: int) -> int:
        """0: window only; 1: one latent per token; r > 1: r tokens pooled per latent.
        Layers past the end of ``compress_ratios`` are window only (config.py:108-111)."""
        r = self.compress_ratios
        return int(r[layer_id]) if 0 <= layer_id < len(r) else 0

    # ---------------------------------------------------------------- sharing topology

    def _resolve_sources(self):
        """Per layer: (kv source or an error message, index source or an error message)."""
        if self._sources is not None:
            return self._sources
        kv_owners = set(self.kv_source_layers)
        index_owners = set(self.index_source_layers)
        depth = max([self.n_layers, len(self.compress_ratios), *(s + 1 for s in kv_owners),
                     *(s + 1 for s in index_owners)])
        latest_kv = latest_index = None
        table = []
        for layer in range(depth):
            if layer in kv_owners:
                latest_kv = layer
            if layer in index_owners:
                latest_index = layer
            if latest_kv is None:
                kv = f"layer {layer} compresses but no kv source layer precedes it"
            elif self.compress_ratio(latest_kv) != self.compress_ratio(layer):
                kv = (f"layer {layer} has compress ratio {self.compress_ratio(layer)}, but its kv "
                      f"source {latest_kv} has ratio {self.compress_ratio(latest_kv)}")
            else:
                kv = latest_kv
            idx = latest_index if latest_index is not None else (
                f"no index source layer precedes layer {layer}")
            table.append((kv, idx))
        self._sources = table
        return table

    def _lookup(self, layer_id: int, which: int) -> int:
        table = self._resolve_sources()
        if not 0 <= layer_id < len(table):
            raise ValueError(f"layer {layer_id} is outside the configured stack")
        found = table[layer_id][which]
        if isinstance(found, str):
            raise ValueError(found)
        return found

    def kv_source_for(self, layer_id: int) -> int:
        """The layer whose compressed-KV cache ``layer_id`` reads: the latest kv source at or
        above it, with an equal compress ratio (config.py:113-127)."""
        return self._lookup(layer_id, 0)

    def index_source_for(self, layer_id: int) -> int:
        """The latest index source at or above ``layer_id`` (config.py:129-133)."""
        return self._lookup(layer_id, 1)

    def __setattr__(self, name, value):
        if name in ("compress_ratios", "kv_source_layers", "index_source_layers", "n_layers"):
            self.__dict__["_sources"] = None
        object.__setattr__(self, name, value)

    # ---------------------------------------------------------------- release files

    @classmethod
    def from_dict(cls, cfg: dict) -> "ModelArgs":
        """Either release layout: the flat inference file or the hub file whose
        ``text_config`` overrides its top level (config.py:135-194)."""
        flat = dict(cfg)
        nested = flat.pop("text_config", None)
        if nested is not None:
            flat.update(nested)
        rope = flat.get("rope_scaling") or {}
        kw = {}
        claimed = {"text_config", "rope_scaling"}
        for name, json_names, _ in _KEYS:
            claimed.update(json_names)
            if name in _FILE_FIXED:
                kw[name] = _FILE_FIXED[name]
                continue
            v = rope.get(_ROPE_SCALING[name]) if name in _ROPE_SCALING else None
            if v is None:
                v = _first(flat, json_names)
            if v is None:
                v = _FILE_DEFAULTS.get(name)
            if v is not None:
                kw[name] = v
        kw.update({k: v for k, v in flat.items() if k not in claimed and k not in _FIELDS})
        return cls(**kw)

    @property
    def raw(self) -> dict:
        """The model type tag of the reference's config (config.py:196-198)."""
        return {"model_type": "deepseek_v41"}
