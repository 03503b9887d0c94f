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
    logits_raw: Optional[torch.Tensor] = None  # [B, vocab] fp32 before the bf16 rounding


def _outputs(out: PrefillResult) -> "capi.AllieOutputs":
    return capi.AllieOutputs(capi.ptr(out.logits).value, capi.ptr(out.value).value, capi.ptr(out.time).value,
                             capi.ptr(out.top1).value, capi.ptr(out.max_logit).value, capi.ptr(out.lse).value,
                             capi.ptr(out.logits_raw).value)


def _new_result(n: int, vocab: int, dev, want_logits: bool, want_raw: bool) -> PrefillResult:
    f = lambda: torch.empty(n, dtype=torch.float32, device=dev)
    lg = lambda: torch.empty(n, vocab, dtype=torch.float32, device=dev)
    return PrefillResult(logits=lg() if want_logits else None, value=f(), time=f(),
                         top1=torch.empty(n, dtype=torch.int32, device=dev), max_logit=f(), lse=f(),
                         logits_raw=lg() if want_raw else None)


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
                kv_block_table: Optional[torch.Tensor] = None,
                out: Optional[PrefillResult] = None, want_raw_logits: bool = False,
                status: Optional[torch.Tensor] = None) -> PrefillResult:
        """Forward of B games given as tokenizer words.

        words: uint32 words of all games back to back (numpy or a device
        tensor of int32/uint32 bits); lens: words per game (host ints).
        legal: optional [B, 62] int32 bitmask over move ids (bit i of word
        i // 32) restricting top1 / lse.
        kv_pool: optional KV pool (``new_kv_pool``) that receives every
        layer's keys and values: game i's position p goes to block
        ``kv_block_table[i, p // 16]`` (device int32 [B, max_blocks]) if that
        table is given, else to the contiguous blocks from ``first_block``.
        status: optional device int32 [1] that receives the packer's flags
        (4: a game longer than its block-table row, 8: the <PAD> id inside a
        game, which is then an ordinary token).
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
            out = _new_result(B, self.cfg.vocab_size, dev, want_logits, want_raw_logits)
        o = _outputs(out)
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
            kv_max_blocks = 0
            if kv_block_table is not None:
                assert kv_block_table.dtype == torch.int32 and kv_block_table.is_contiguous()
                assert kv_block_table.shape[0] == B
                kv_max_blocks = kv_block_table.shape[1]
            rc = self._lib.allie_prefill(
                self._m, capi.ptr(wd), lens_np.ctypes.data_as(C.c_void_p), B, float(temperature),
                capi.ptr(legal_t), LEGAL_WORDS if legal_t is not None else 0, C.byref(o),
                capi.ptr(kv_pool), int(kv_blocks), int(first_block), capi.ptr(kv_block_table),
                int(kv_max_blocks), capi.ptr(status), capi.ptr(ws), ws.numel(), capi.stream_ptr(),
            )
            capi.check(rc, "allie_prefill")
        return out

    # ------------------------------------------------------------- KV cache
    def new_kv_pool(self, n_blocks: int) -> torch.Tensor:
        """Device KV pool of n_blocks blocks of 16 positions (every layer's
        keys and values, layout [layer][block][k|v][head][16][64])."""
        return torch.empty(n_blocks * self.kv_block_bytes(), dtype=torch.uint8, device=self.device)

    def pool_blocks(self, kv_pool: torch.Tensor) -> int:
        return kv_pool.numel() * kv_pool.element_size() // self.kv_block_bytes()

    # --------------------------------------------------------------- extend
    def extend(self, ids, pos, group_sizes, prefix_len, prefix_blocks, extra_slot, n_extra,
               kv_pool: torch.Tensor, temperature: float = 1.0, legal=None, want_logits: bool = True,
               status: Optional[torch.Tensor] = None, out: Optional[PrefillResult] = None,
               noalloc: bool = False, want_raw_logits: bool = False) -> PrefillResult:
        """Forward of n new tokens over the paged KV cache (decode steps, MCTS
        tree levels).  Tokens come in groups of ``group_sizes`` (host ints);
        token i of group g attends the group's prefix (``prefix_len[g]``
        positions in blocks ``prefix_blocks[g]``) and then its own pool slots
        ``extra_slot[i, :n_extra[i]]``, the last of which receives its keys and
        values.  Array arguments are device int32 tensors (or numpy, copied).
        Returns per-token outputs like ``prefill``.

        noalloc: run through ``allie_extend_noalloc`` (no workspace; the
        library's per-device scratch, at most 256 tokens), which takes the
        group starts as a device array."""
        dev = self.device

        def dt(a, shape=None):
            t = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32))
            t = t.to(device=dev, dtype=torch.int32).contiguous()
            return t if shape is None else t.reshape(shape)

        gs = np.asarray(group_sizes, dtype=np.int64)
        G = len(gs)
        n = int(gs.sum())
        group_start = np.zeros(G + 1, dtype=np.int32)
        group_start[1:] = np.cumsum(gs)
        ids_t, pos_t = dt(ids), dt(pos)
        pl_t = dt(prefix_len)
        pb_t = dt(prefix_blocks)
        pb_t = pb_t.reshape(G, -1) if pb_t.numel() else pb_t.reshape(G, 0)
        es_t = dt(extra_slot).reshape(n, -1)
        ne_t = dt(n_extra)
        assert ids_t.numel() == n and pos_t.numel() == n and ne_t.numel() == n and pl_t.numel() == G
        if out is None:
            out = _new_result(n, self.cfg.vocab_size, dev, want_logits, want_raw_logits)
        o = _outputs(out)
        with torch.cuda.device(dev):
            legal_t = None
            if legal is not None:
                legal_t = _as_tensor(legal).to(torch.int32).to(dev).contiguous()
                assert legal_t.shape == (n, LEGAL_WORDS)
            if noalloc:
                gs_t = torch.from_numpy(group_start).to(dev)
                rc = self._lib.allie_extend_noalloc(
                    self._m, capi.ptr(ids_t), capi.ptr(pos_t), n, group_start.ctypes.data_as(C.c_void_p),
                    capi.ptr(gs_t), G, capi.ptr(pl_t), capi.ptr(pb_t), pb_t.shape[1], capi.ptr(es_t), capi.ptr(ne_t),
                    es_t.shape[1], float(temperature), capi.ptr(legal_t), LEGAL_WORDS if legal_t is not None else 0,
                    C.byref(o), capi.ptr(kv_pool), self.pool_blocks(kv_pool), capi.ptr(status), capi.stream_ptr(),
                )
                capi.check(rc, "allie_extend_noalloc")
                return out
            ws = self._workspace(int(self._lib.allie_extend_workspace_bytes(self._m, n, G)))
            rc = self._lib.allie_extend(
                self._m, capi.ptr(ids_t), capi.ptr(pos_t), n, group_start.ctypes.data_as(C.c_void_p), G,
                capi.ptr(pl_t), capi.ptr(pb_t), pb_t.shape[1], capi.ptr(es_t), capi.ptr(ne_t), es_t.shape[1],
                float(temperature), capi.ptr(legal_t), LEGAL_WORDS if legal_t is not None else 0, C.byref(o),
                capi.ptr(kv_pool), self.pool_blocks(kv_pool), capi.ptr(status), capi.ptr(ws), ws.numel(),
                capi.stream_ptr(),
            )
            capi.check(rc, "allie_extend")
        return out

    def extend_noalloc_raw(self, ids, pos, group_start_host: np.ndarray, group_start, prefix_len, prefix_blocks,
                           extra_slot, n_extra, kv_pool: torch.Tensor, out: PrefillResult,
                           status: torch.Tensor, temperature: float = 1.0) -> None:
        """``allie_extend_noalloc`` on device int32 tensors the caller owns
        (``prefix_blocks`` [G, max_blocks], ``extra_slot`` [n, max_extra]) and
        a preallocated ``out``: no tensor is created and nothing is copied, so
        the call can be captured into a HIP graph and replayed with new
        contents in the same buffers."""
        G = len(group_start_host) - 1
        n = int(group_start_host[-1])
        o = _outputs(out)
        rc = self._lib.allie_extend_noalloc(
            self._m, capi.ptr(ids), capi.ptr(pos), n, group_start_host.ctypes.data_as(C.c_void_p),
            capi.ptr(group_start), G, capi.ptr(prefix_len), capi.ptr(prefix_blocks), prefix_blocks.shape[1],
            capi.ptr(extra_slot), capi.ptr(n_extra), extra_slot.shape[1], float(temperature), None, 0, C.byref(o),
            capi.ptr(kv_pool), self.pool_blocks(kv_pool), capi.ptr(status), capi.stream_ptr())
        capi.check(rc, "allie_extend_noalloc")

    def set_split_tokens(self, tokens: int, decode_tokens: int = 512) -> None:
        """Thresholds of the two-stream split of large bf16 prefills and
        extends, and of extends with many one-token groups
        (``allie_model_set_split_tokens``); 0 turns a split off."""
        capi.check(self._lib.allie_model_set_split_tokens(self._m, int(tokens), int(decode_tokens)),
                   "allie_model_set_split_tokens")

    def set_tree_heads(self, heads: int) -> None:
        """Heads per tree-attention workgroup (``allie_model_set_tree_heads``):
        0 chooses by the launch size; the results are the same bits either way."""
        capi.check(self._lib.allie_model_set_tree_heads(self._m, int(heads)), "allie_model_set_tree_heads")

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
