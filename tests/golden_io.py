"""Reading and writing the golden fixtures in tests/golden (npz, no pickles): case parameters as JSON text,
inputs as bf16 bit patterns, expected O / LSE as float64."""
import json

import numpy as np

import fmha_cases as FC


def save(path, case: FC.Case, arrays: dict, o, lse):
    meta = dict(name=case.name, B=case.B, S=case.S, N=case.N, Hq=case.Hq, Hkv=case.Hkv, D=case.D, mode=case.mode,
                seed=case.seed, seqlens=list(case.seqlens))
    payload = {f"in_{k}": v for k, v in arrays.items()}
    np.savez_compressed(path, meta=np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8), o=o, lse=lse, **payload)


def load(path):
    z = np.load(path, allow_pickle=False)
    meta = json.loads(bytes(z["meta"]).decode())
    arrays = {k[3:]: z[k] for k in z.files if k.startswith("in_")}
    qpos = arrays.get("qpos")
    case = FC.Case(meta["name"], B=meta["B"], S=meta["S"], N=meta["N"], Hq=meta["Hq"], Hkv=meta["Hkv"], D=meta["D"],
                   mode=meta["mode"], seed=meta["seed"], seqlens=meta["seqlens"],
                   qpos=qpos if meta["mode"] == "qpos" else None)
    return case, arrays, z["o"], z["lse"]
