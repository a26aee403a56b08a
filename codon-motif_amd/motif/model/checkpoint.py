'''Weights on disk: reading and writing MotifChord checkpoints.

Same surface as the reference's motif/model/checkpoint.py (`load_checkpoint`
:716-760, `config_from_state_dict` :441-558, `strip_wrapper_prefixes` :578-602,
`save_safetensors` :263-368, `config_from_mapping` :371-392, `config_to_dict`
:219-230): a bare state_dict, a training-pipeline checkpoint (a mapping whose
`payload['model']` holds the weights) or safetensors (one file, a shard directory
or an `*.index.json`) come back as canonical weight names plus whatever config the
file carried; `config_from_state_dict` recovers the hyper-parameters from the
tensor shapes when it carried none.

One deliberate difference: `.pt` files are read with `torch.load(weights_only=True)`
only.  The reference falls back to the full unpickler, which executes code stored
in the file; a checkpoint that needs it is refused here with the loader's error.
'''
import json
import os
import re
from dataclasses import asdict, dataclass, field, fields
from typing import Any, Dict, List, Optional, Tuple, Union

import torch
import torch.nn as nn

from .config import MotifChordConfig

try:
    from safetensors import safe_open
    from safetensors.torch import load_file as _st_load
    from safetensors.torch import save_file as _st_save
    HAS_SAFETENSORS = True
except ImportError:  # pragma: no cover - the image ships safetensors
    safe_open = _st_load = _st_save = None
    HAS_SAFETENSORS = False

# Wrapper prefixes that training wrappers put in front of every key (DDP, torch.compile,
# FSDP, activation checkpointing, a `model` attribute).
WRAPPER_PREFIXES = ('module.', '_orig_mod.', '_forward_module.', '_checkpoint_wrapped_module.', 'model.')
# Mapping keys under which a checkpoint may keep its config.
CONFIG_KEYS = ('config', 'model_config', 'motif_config', 'modelconfig', 'config_dict')
# Common names of other configuration formats for MotifChordConfig fields.
CONFIG_ALIASES = {
    'hidden_size': 'model_dim', 'd_model': 'model_dim', 'n_embd': 'model_dim',
    'num_hidden_layers': 'block_n', 'n_layers': 'block_n', 'num_layers': 'block_n',
    'num_attention_heads': 'num_heads', 'n_heads': 'num_heads',
    'num_key_value_heads': 'num_kv_heads', 'n_kv_heads': 'num_kv_heads',
}
_FIELDS = {f.name for f in fields(MotifChordConfig)}


@dataclass
class LoadedCheckpoint:
    '''Weights (canonical names) plus the config found in the file (None: infer it).'''
    state_dict: Dict[str, torch.Tensor]
    config: Optional[MotifChordConfig]
    source: str
    path: str
    metadata: Dict[str, str] = field(default_factory=dict)


def looks_like_safetensors(path: str) -> bool:
    '''True when the file starts with a safetensors header (a little-endian u64 length,
    then a JSON object), whatever its name.'''
    if path.endswith('.safetensors'):
        return True
    if path.endswith('.index.json') or os.path.isdir(path):
        return False
    try:
        size = os.path.getsize(path)
        with open(path, 'rb') as fh:
            head = fh.read(8)
            if len(head) < 8:
                return False
            n = int.from_bytes(head, 'little')
            if n <= 0 or n > (1 << 28) or 8 + n > size:
                return False
            return fh.read(min(n, 32)).lstrip()[:1] == b'{'
    except OSError:
        return False


def config_to_dict(config: MotifChordConfig) -> Dict[str, Any]:
    '''Plain JSON-compatible fields (tuples as lists).'''
    return {k: list(v) if isinstance(v, tuple) else v for k, v in asdict(config).items()}


def config_from_mapping(spec: Dict[str, Any]) -> MotifChordConfig:
    '''MotifChordConfig from a mapping; aliases are translated, unknown keys ignored.'''
    out = {}
    for key, value in spec.items():
        name = CONFIG_ALIASES.get(key, key)
        if name in _FIELDS:
            out[name] = tuple(value) if name == 'block' and isinstance(value, list) else value
    return MotifChordConfig(**out)


def _as_config(value: Any) -> Optional[MotifChordConfig]:
    if value is None:
        return None
    if isinstance(value, MotifChordConfig):
        return value
    if isinstance(value, (str, bytes)):
        try:
            value = json.loads(value)
        except (TypeError, ValueError):
            return None
    return config_from_mapping(value) if isinstance(value, dict) else None


def _find_config(*containers: Any) -> Optional[MotifChordConfig]:
    for c in containers:
        if isinstance(c, dict):
            for key in CONFIG_KEYS:
                cfg = _as_config(c.get(key))
                if cfg is not None:
                    return cfg
    return None


def strip_wrapper_prefixes(sd: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    '''Drop wrapper prefixes while every key carries the same one.'''
    out = dict(sd)
    while out:
        for prefix in WRAPPER_PREFIXES:
            if all(k.startswith(prefix) for k in out):
                out = {k[len(prefix):]: v for k, v in out.items()}
                break
        else:
            break
    return out


def config_from_state_dict(sd: Dict[str, torch.Tensor]) -> MotifChordConfig:
    '''Hyper-parameters from the tensor shapes of canonical-name weights.

    vocab / model_dim from `embed.weight` (or `lm_head.weight`); `block_n` from the
    largest `blocks.<n>.`; the recipe from block 0's layers (`theta_alpha`: chord,
    `a_proj` / `q_conv`: gdn); heads from the per-head vectors; kv heads from a chord
    layer's `k_proj`; `head_k_dim` from a gdn layer's `q_proj` (64 when no gdn layer
    exists); `tied_weight` from whether the head equals the embedding.
    '''
    emb = sd.get('embed.weight', sd.get('lm_head.weight'))
    if emb is None:
        raise ValueError("cannot infer the config: no 'embed.weight' or 'lm_head.weight'.")
    if emb.dim() != 2:
        raise ValueError(f"cannot infer the config: 'embed.weight' has shape {tuple(emb.shape)}.")
    vocab, dim = int(emb.shape[0]), int(emb.shape[1])
    blocks = sorted({int(m.group(1)) for k in sd if (m := re.match(r'blocks\.(\d+)\.', k))})
    if not blocks:
        raise ValueError("cannot infer the config: no 'blocks.<n>.' keys.")
    layers = sorted({int(m.group(1)) for k in sd if (m := re.match(r'blocks\.0\.features\.(\d+)\.', k))})
    if not layers:
        raise ValueError("cannot infer the config: block 0 has no 'features.<n>.' keys.")
    recipe: List[str] = []
    heads = kv_heads = head_k = None
    for i in layers:
        p = f'blocks.0.features.{i}.attn.'
        if p + 'theta_alpha' in sd:
            recipe.append('chord')
            n = int(sd[p + 'theta_alpha'].shape[0])
            heads = heads or n
            kw = sd.get(p + 'k_proj.weight')
            if kw is not None and dim // n > 0:
                kv_heads = int(kw.shape[0]) // (dim // n)
        elif p + 'a_proj.weight' in sd or p + 'a_proj' in sd or p + 'q_conv.weight' in sd:
            recipe.append('gdn')
            anchor = sd.get(p + 'a_proj.weight', sd.get(p + 'A_log'))
            if anchor is not None:
                heads = heads or int(anchor.shape[0])
            qw = sd.get(p + 'q_proj.weight')
            if qw is not None and heads:
                head_k = int(qw.shape[0]) // heads
        else:
            raise ValueError(f"cannot infer the config: {p} has neither chord ('theta_alpha') nor "
                             f"gated delta-net ('q_conv' / 'a_proj') weights.")
    if heads is None:
        raise ValueError('cannot infer the config: no per-head parameter found.')
    head = sd.get('lm_head.weight')
    tied = head is None or head is emb or (head.shape == emb.shape and (
        (head.device == emb.device and head.data_ptr() == emb.data_ptr()) or torch.equal(head, emb)))
    return MotifChordConfig(vocab_size=vocab, model_dim=dim, num_heads=heads,
                            num_kv_heads=kv_heads if kv_heads is not None else heads,
                            head_k_dim=head_k if head_k is not None else 64, tied_weight=bool(tied),
                            block=tuple(recipe), block_n=blocks[-1] + 1)


def _shards(path: str) -> Tuple[List[str], Optional[str]]:
    '''Safetensors files to read and the `config.json` beside them (if any).'''
    def sidecar(d):
        c = os.path.join(d, 'config.json')
        return c if os.path.isfile(c) else None
    if path.endswith('.index.json'):
        d = os.path.dirname(os.path.abspath(path))
        with open(path, 'r', encoding='utf-8') as fh:
            names = sorted(set((json.load(fh).get('weight_map') or {}).values()))
        if not names:
            raise FileNotFoundError(f'{path} lists no weight shards.')
        return [os.path.join(d, n) for n in names], sidecar(d)
    if os.path.isdir(path):
        d = os.path.abspath(path)
        one = os.path.join(d, 'model.safetensors')
        if os.path.isfile(one):
            return [one], sidecar(d)
        files = sorted(os.path.join(d, n) for n in os.listdir(d) if n.endswith('.safetensors'))
        if not files:
            raise FileNotFoundError(f'no .safetensors file under {path!r}.')
        return files, sidecar(d)
    return [os.path.abspath(path)], sidecar(os.path.dirname(os.path.abspath(path)))


def _from_torch_object(obj: Any, path: str) -> LoadedCheckpoint:
    def wrap(src, sd, cfg):
        return LoadedCheckpoint(strip_wrapper_prefixes(sd), cfg, src, path)

    def tensor_dict(v):
        return isinstance(v, dict) and len(v) > 0 and all(isinstance(t, torch.Tensor) for t in v.values())

    if isinstance(obj, nn.Module):
        return wrap('nn.Module', obj.state_dict(), None)
    if not isinstance(obj, dict):
        raise ValueError(f'{path!r} holds {type(obj).__name__}, expected a state_dict or a checkpoint mapping.')
    payload = obj.get('payload')
    if isinstance(payload, dict):
        model = payload.get('model')
        if tensor_dict(model):
            return wrap(f"pipeline checkpoint ({obj.get('__pipeline__') or 'pipeline'!r})", model,
                        _find_config(obj, payload))
    for key in ('state_dict', 'model_state_dict', 'weights', 'model'):
        if tensor_dict(obj.get(key)):
            return wrap(f'state_dict under {key!r}', obj[key], _find_config(obj))
    tensors = {k: v for k, v in obj.items() if isinstance(v, torch.Tensor)}
    if tensors:
        return wrap('bare state_dict', tensors, _find_config(obj))
    raise ValueError(f'cannot find model weights in {path!r}: keys {sorted(obj)[:8]}.')


def load_checkpoint(path: str, map_location: Any = 'cpu') -> LoadedCheckpoint:
    '''Read a bare state_dict, a pipeline checkpoint or safetensors (file, shard
    directory, `*.index.json`, or a directory holding one of those).'''
    path = os.fspath(path)
    if not os.path.exists(path):
        raise FileNotFoundError(f'checkpoint not found: {path!r}')
    if os.path.isdir(path) or looks_like_safetensors(path) or path.endswith('.index.json'):
        if os.path.isdir(path) and not any(n.endswith(('.safetensors', '.index.json')) for n in os.listdir(path)):
            for name in ('last.pt', 'model.pt', 'pytorch_model.bin'):
                if os.path.isfile(os.path.join(path, name)):
                    return load_checkpoint(os.path.join(path, name), map_location)
        if not HAS_SAFETENSORS:
            raise ImportError('reading a safetensors checkpoint needs the `safetensors` package.')
        files, side = _shards(path)
        sd: Dict[str, torch.Tensor] = {}
        meta: Dict[str, str] = {}
        for f in files:
            sd.update(_st_load(f, device=str(map_location)))
            with safe_open(f, framework='pt', device='cpu') as fh:
                meta.update(fh.metadata() or {})
        cfg = _find_config(meta)
        if cfg is None and side is not None:
            with open(side, 'r', encoding='utf-8') as fh:
                cfg = _as_config(json.load(fh))
        return LoadedCheckpoint(strip_wrapper_prefixes(sd), cfg, 'safetensors', path, meta)
    try:
        obj = torch.load(path, map_location=map_location, weights_only=True)
    except Exception as exc:
        raise ValueError(f'{path!r} cannot be read with torch.load(weights_only=True) (files that '
                         f'need the full unpickler are not loaded): {exc}') from exc
    return _from_torch_object(obj, path)


def save_safetensors(model_or_state: Any, path: str,
                     config: Optional[Union[MotifChordConfig, Dict[str, Any]]] = None,
                     metadata: Optional[Dict[str, Any]] = None) -> Dict[str, Any]:
    '''Write weights (a module, a state_dict or a checkpoint path) and their config
    (JSON under the `'config'` metadata key) to one `.safetensors` file.  An
    `lm_head.weight` sharing storage with `embed.weight` is written once.'''
    if not HAS_SAFETENSORS:
        raise ImportError('writing a safetensors checkpoint needs the `safetensors` package.')
    source = 'state_dict'
    cfg = config if isinstance(config, MotifChordConfig) else None
    if isinstance(config, dict):
        cfg = config_from_mapping(config)
    if isinstance(model_or_state, (str, os.PathLike)):
        loaded = load_checkpoint(os.fspath(model_or_state))
        sd, source = loaded.state_dict, loaded.source
        cfg = cfg or loaded.config
    elif isinstance(model_or_state, nn.Module):
        sd, source = model_or_state.state_dict(), type(model_or_state).__name__
        cfg = cfg or getattr(model_or_state, 'config', None)
    elif isinstance(model_or_state, dict):
        sd = model_or_state
    else:
        raise ValueError(f'cannot save {type(model_or_state).__name__}: expected a module, a state_dict or a path.')
    if not sd:
        raise ValueError('no weights to save.')
    cfg = cfg or config_from_state_dict(sd)
    emb, head = sd.get('embed.weight'), sd.get('lm_head.weight')
    dropped = []
    if emb is not None and head is not None and (head is emb or (
            head.data_ptr() == emb.data_ptr() and head.shape == emb.shape and head.device == emb.device)):
        dropped = ['lm_head.weight']
    out = {}
    for k, v in sd.items():
        if k in dropped:
            continue
        if not isinstance(v, torch.Tensor):
            raise ValueError(f'{k!r} is not a tensor ({type(v).__name__}).')
        out[k] = v.detach().to('cpu').contiguous()
    info = {'format': 'pt', 'producer': 'motif-checkpoint/1',
            'config': json.dumps(config_to_dict(cfg), ensure_ascii=False)}
    for k, v in (metadata or {}).items():
        info[str(k)] = v if isinstance(v, str) else json.dumps(v, ensure_ascii=False)
    path = os.fspath(path)
    d = os.path.dirname(os.path.abspath(path))
    if not os.path.isdir(d):
        raise FileNotFoundError(f'destination directory does not exist: {d!r}')
    _st_save(out, path, metadata=info)
    return {'path': path, 'source': source, 'tensors': len(out),
            'params': int(sum(v.numel() for v in out.values())), 'bytes': os.path.getsize(path),
            'config': config_to_dict(cfg), 'dropped': dropped, 'metadata': info}
