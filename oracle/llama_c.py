"""ctypes wrapper of the C Llama decoder + greedy loop (test infrastructure).

``oracle/c/strata_oracle_llama.c`` restates ``oracle/llama.py``'s model and
``greedy_generate`` (``src/ollm/llama_mlx.py:53-912``,
``src/ollm/generation.py:7-50``) in plain C with OpenMP, so that full-depth
models (28 layers, vocab 128256) run in seconds on the CPU.  It is pinned
against ``OracleLlama`` on tiny configs in ``tests/test_oracle_llama_c.py``
(identical greedy ids and float32-level logits).  Weights use
``OracleLlama``'s names: q4 triples for the seven linears of each layer,
bf16 ``embed_tokens``, ``norm``, the two layer norms and a bf16 ``lm_head``
(absent: tied to the embedding).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path
from typing import Dict, Optional, Tuple

import numpy as np

_SO = Path(__file__).resolve().parent / "libstrata_oracle.so"
_LIN = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
_P = C.c_void_p


class _Model(C.Structure):
    _fields_ = [("vocab", C.c_int), ("hidden", C.c_int), ("ffn", C.c_int), ("layers", C.c_int),
                ("heads", C.c_int), ("kv_heads", C.c_int), ("group", C.c_int),
                ("eps", C.c_float), ("theta", C.c_float),
                ("embed", _P), ("norm", _P), ("lm_head", _P),
                ("ln1", C.POINTER(_P)), ("ln2", C.POINTER(_P)),
                ("w", C.POINTER(_P)), ("s", C.POINTER(_P)), ("b", C.POINTER(_P))]


def _lib():
    if not _SO.exists():
        raise FileNotFoundError(f"{_SO} not built (make -C oracle/c)")
    lib = C.CDLL(str(_SO))
    lib.oracle_llama_generate.argtypes = [C.POINTER(_Model), _P, C.c_int, C.c_int, _P, _P, _P]
    lib.oracle_llama_generate.restype = C.c_int
    lib.oracle_llama_set_f32_accum.argtypes = [C.c_int]
    return lib


class CLlama:
    """C decoder over host weights (``cfg`` has ``oracle.llama.Config``'s fields)."""

    def __init__(self, cfg, weights: Dict[str, np.ndarray]):
        if "lm_head.weight" in weights or "embed_tokens.weight" in weights:
            raise ValueError("the C decoder takes a bf16 embedding and lm_head")
        self.cfg = cfg
        keep = {}

        def arr(name, dtype):
            a = np.ascontiguousarray(weights[name]).view(dtype)
            keep[name] = a
            return a.ctypes.data

        L = cfg.num_hidden_layers
        ln1 = (_P * L)(*[arr(f"layers.{i}.input_layernorm", np.uint16) for i in range(L)])
        ln2 = (_P * L)(*[arr(f"layers.{i}.post_attention_layernorm", np.uint16) for i in range(L)])
        ws, ss, bs = (_P * (7 * L))(), (_P * (7 * L))(), (_P * (7 * L))()
        for i in range(L):
            for j, n in enumerate(_LIN):
                p = f"layers.{i}.{n}"
                ws[7 * i + j] = arr(p + ".weight", np.uint32)
                ss[7 * i + j] = arr(p + ".scales", np.uint16)
                bs[7 * i + j] = arr(p + ".biases", np.uint16)
        self._keep = (keep, ln1, ln2, ws, ss, bs)
        self._m = _Model(cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, L,
                         cfg.num_attention_heads, cfg.num_key_value_heads, cfg.group_size,
                         cfg.rms_norm_eps, cfg.rope_theta,
                         arr("embed_tokens", np.uint16), arr("norm", np.uint16),
                         arr("lm_head", np.uint16) if "lm_head" in weights else None,
                         ln1, ln2, ws, ss, bs)
        self._lib = _lib()

    def set_f32_accum(self, on: bool) -> None:
        """Switch the linears to fp32 accumulation (an accumulation-order probe:
        ids that change under it are ill-conditioned for bit-exact checks)."""
        self._lib.oracle_llama_set_f32_accum(1 if on else 0)

    def generate(self, prompt, max_new_tokens: int) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
        """Greedy ids ``[n_prompt + max_new]``, per-token top-1/top-2 logit
        margins ``[max_new]`` and the logits that chose the last token."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int64).reshape(-1))
        ids = np.zeros(p.size + max_new_tokens, dtype=np.int64)
        margins = np.zeros(max(max_new_tokens, 1), dtype=np.float32)
        logits = np.zeros(self.cfg.vocab_size, dtype=np.float32)
        rc = self._lib.oracle_llama_generate(C.byref(self._m), p.ctypes.data, int(p.size),
                                             int(max_new_tokens), ids.ctypes.data,
                                             margins.ctypes.data, logits.ctypes.data)
        if rc != 0:
            raise ValueError("oracle_llama_generate rejected its arguments")
        return ids, margins[:max_new_tokens], logits


def generate(cfg, weights: Dict[str, np.ndarray], prompt, max_new_tokens: int,
             model: Optional[CLlama] = None):
    return (model or CLlama(cfg, weights)).generate(prompt, max_new_tokens)
