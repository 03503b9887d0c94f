"""Engine: the device-resident model and its batched entry points.

``Engine`` owns one ``allie_model`` of the C ABI (weights packed into a
device arena) and the workspaces its calls need.  Its calls replace, for a
whole batch at once, what the reference does per game:

* ``prefill(words, lens)`` -- ``model(**tokenizer.pad_and_collate(games))``
  followed by the last-token reads of ``Policy.score_full``
  (src/evaluation/decode.py:199-226): returns per-game logits, value, time,
  the first argmax over the (legal) move logits and their logsumexp.

Everything is stream-ordered on torch's current stream; outputs are torch
tensors on the engine's device.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import capi
from . import weights as W
from .config import BF16, FP8W, FP32, ModelConfig

_GLOBAL_KINDS = {
    "wte": capi.W_WTE, "wpe": capi.W_WPE, "ctrl": capi.W_CTRL, "lnf_g": capi.W_LNF_G,
    "lnf_b": capi.W_LNF_B, "w_value": capi.W_VALUE_W, "b_value": capi.W_VALUE_B,
    "w_time": capi.W_TIME_W, "b_time": capi.W_TIME_B,
}
_LAYER_KINDS = {
    "ln1_g": capi.W_LN1_G, "ln1_b": capi.W_LN1_B, "w_qkv": capi.W_QKV_W, "b_qkv": capi.W_QKV_B,
    "w_o": capi.W_O_W, "b_o": capi.W_O_B, "ln2_g": capi.W_LN2_G, "ln2_b": capi.W_LN2_B,
    "w_fc": capi.W_FC_W, "b_fc": capi.W_FC_B, "w_pr": capi.W_PR_W, "b_pr": capi.W_PR_B,
}
_GEMM_WEIGHTS = ("w_qkv", "w_o", "w_fc", "w_pr")

N_MOVES = 1968
LEGAL_WORDS = (N_MOVES + 31) // 32


@dataclass
class PrefillResult:
    logits: Optional[torch.Tensor]  # [B, vocab] fp32 (bf16-rounded values in bf16 modes)
    value: torch.Tensor             # [B]
    time: torch.Tensor              # [B]
    top1: torch.Tensor              # [B] int32
    max_logit: torch.Tensor         # [B]
    lse: torch.Tensor               # [B]


def _as_tensor(a) -> torch.Tensor:
    if isinstance(a, torch.Tensor):
        return a
    return torch.from_numpy(np.ascontiguousarray(a))


class Engine:
    def __init__(self, cfg: ModelConfig, state_dict: dict, mode: str = BF16, device: str = "cuda:0"):
        if mode not in (FP32, BF16, FP8W):
            raise ValueError(f"unknown mode {mode}")
        if not torch.cuda.is_available():
            raise capi.AllieError("the engine needs a ROCm GPU (no CPU fallback)")
        self.cfg, self.mode = cfg, mode
        self.device = torch.device(device)
        self._lib = capi.lib()
        c = capi.AllieConfig(cfg.n_layer, cfg.d_model, cfg.n_head, cfg.vocab_size, cfg.n_positions,
                             cfg.max_length, cfg.eps, capi.MODE_IDS[mode])
        h = C.c_void_p()
        with torch.cuda.device(self.device):
            capi.check(self._lib.allie_model_create(C.byref(c), C.byref(h)), "allie_model_create")
        self._m = h
        self._ws = None
        try:
            self._load(state_dict)
        except Exception:
            self.close()
            raise

    # -------------------------------------------------------------- weights
    def _load(self, sd: dict) -> None:
        L = self._lib
        with torch.cuda.device(self.device):
            st = capi.stream_ptr()
            keep = []  # device staging tensors live until the stream has consumed them

            def put(kind, layer, arr):
                t = _as_tensor(arr).to(torch.float32).contiguous()
                rows, cols = (t.shape[0], t.shape[1]) if t.dim() == 2 else (1, t.numel())
                td = t.to(self.device)
                keep.append(td)
                capi.check(L.allie_model_set_weight(self._m, kind, layer, capi.ptr(td), rows, cols, st),
                           f"set_weight({kind}, {layer})")

            for name, kind in _GLOBAL_KINDS.items():
                put(kind, 0, sd[W.GLOBAL_KEYS[name]])
            for i in range(self.cfg.n_layer):
                keys = W.layer_keys(i)
                for name, kind in _LAYER_KINDS.items():
                    arr = sd[keys[name]]
                    if self.mode == FP8W and name in _GEMM_WEIGHTS:
                        a = arr.numpy() if isinstance(arr, torch.Tensor) else np.asarray(arr)
                        q, s = W.quantize_fp8_per_channel(a)
                        qd = torch.from_numpy(q).to(self.device)
                        sdv = torch.from_numpy(s).to(self.device)
                        keep += [qd, sdv]
                        capi.check(L.allie_model_set_weight_fp8(self._m, kind, i, capi.ptr(qd), capi.ptr(sdv),
                                                                q.shape[0], q.shape[1], st),
                                   f"set_weight_fp8({name}, {i})")
                    else:
                        put(kind, i, arr)
            torch.cuda.current_stream().synchronize()
            del keep
            capi.check(L.allie_model_finalize(self._m), "allie_model_finalize")

    # ------------------------------------------------------------ workspace
    def _workspace(self, nbytes: int) -> torch.Tensor:
        if self._ws is None or self._ws.numel() < nbytes:
            self._ws = None
            self._ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=self.device)
        return self._ws

    def prefill_workspace_bytes(self, n_seq: int, n_tokens: int) -> int:
        return int(self._lib.allie_prefill_workspace_bytes(self._m, n_seq, n_tokens))

    def kv_block_bytes(self) -> int:
        return int(self._lib.allie_kv_block_bytes(self._m))

    # -------------------------------------------------------------- prefill
    def prefill(self, words, lens, temperature: float = 1.0, legal=None, want_logits: bool = True,
                kv_pool: Optional[torch.Tensor] = None, first_block: int = 0,
                out: Optional[PrefillResult] = None) -> PrefillResult:
        """Forward of B games given as tokenizer words.

        words: uint32 words of all games back to back (numpy or a device
        tensor of int32/uint32 bits); lens: words per game (host ints).
        legal: optional [B, 62] int32 bitmask over move ids (bit i of word
        i // 32) restricting top1 / lse.
        """
        lens_np = np.ascontiguousarray(np.asarray(lens, dtype=np.int32))
        B = len(lens_np)
        dev = self.device
        if isinstance(words, torch.Tensor) and words.is_cuda:
            wd = words.view(torch.int32) if words.dtype != torch.int32 else words
        else:
            wd = torch.from_numpy(np.ascontiguousarray(np.asarray(words, dtype=np.uint32)).view(np.int32)).to(dev)
        n = np.minimum(lens_np, self.cfg.max_length)
        T = int(n.sum())
        if out is None:
            f = lambda: torch.empty(B, dtype=torch.float32, device=dev)
            out = PrefillResult(
                logits=torch.empty(B, self.cfg.vocab_size, dtype=torch.float32, device=dev) if want_logits else None,
                value=f(), time=f(), top1=torch.empty(B, dtype=torch.int32, device=dev),
                max_logit=f(), lse=f(),
            )
        o = capi.AllieOutputs(capi.ptr(out.logits).value, capi.ptr(out.value).value, capi.ptr(out.time).value,
                              capi.ptr(out.top1).value, capi.ptr(out.max_logit).value, capi.ptr(out.lse).value)
        ws_bytes = self.prefill_workspace_bytes(B, T)
        with torch.cuda.device(dev):
            ws = self._workspace(ws_bytes)
            legal_t = None
            if legal is not None:
                legal_t = _as_tensor(legal).to(torch.int32).to(dev).contiguous()
                assert legal_t.shape == (B, LEGAL_WORDS)
            kv_blocks = 0
            if kv_pool is not None:
                kv_blocks = kv_pool.numel() * kv_pool.element_size() // self.kv_block_bytes()
            rc = self._lib.allie_prefill(
                self._m, capi.ptr(wd), lens_np.ctypes.data_as(C.c_void_p), B, float(temperature),
                capi.ptr(legal_t), LEGAL_WORDS if legal_t is not None else 0, C.byref(o),
                capi.ptr(kv_pool), int(kv_blocks), int(first_block), capi.ptr(ws), ws.numel(),
                capi.stream_ptr(),
            )
            capi.check(rc, "allie_prefill")
        return out

    def close(self) -> None:
        if getattr(self, "_m", None):
            self._lib.allie_model_destroy(self._m)
            self._m = None
        self._ws = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def legal_mask(legal_ids_per_game: list, n_moves: int = N_MOVES) -> np.ndarray:
    """[B, 62] int32 bitmask from lists of legal move ids."""
    m = np.zeros((len(legal_ids_per_game), LEGAL_WORDS), dtype=np.uint32)
    for b, ids in enumerate(legal_ids_per_game):
        for i in ids:
            if 0 <= i < n_moves:
                m[b, i >> 5] |= np.uint32(1) << np.uint32(i & 31)
    return m.view(np.int32)
