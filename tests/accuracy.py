"""Teacher-forcing accuracy harness for the decode driver (the reference's real-model check,
app/llm_real.cpp:292-343 in arasheedu/Kernelcore).

The reference compares its engine with llama.cpp's greedy run of a real model: the same top token
at every generated position, |log-prob difference| of llama.cpp's token (mean and max), top-5
overlap, and how many tokens a free greedy run keeps identical. No model file or llama.cpp ships
here, so the reference run is the CPU oracle model (oracle/model.py) on the same random weights:
its greedy continuation of a prompt gives the token sequence, its log-probs and its top-5 lists.
Every position is fed as a single token (the reference's decodeToken loop), so the numbers
measure the single-token decode path; `free_run` also covers the graph-replayed generate.
"""
import numpy as np


def log_softmax(logits):
    z = np.asarray(logits, np.float64)
    z = z - z.max()
    return z - np.log(np.exp(z).sum())


def reference_run(oracle, prompt, n_gen, k_top=5):
    """The oracle's greedy continuation: per generated token its id, log-prob and the top-k ids."""
    logits = None
    for t in prompt:
        logits = oracle.forward([int(t)])
    gen = []
    for i in range(n_gen):
        ls = log_softmax(logits)
        tok = int(np.argmax(logits))
        top = [int(j) for j in np.argsort(-np.asarray(logits, np.float64), kind="stable")[:k_top]]
        gen.append({"id": tok, "logprob": float(ls[tok]), "top": top})
        if i + 1 < n_gen:
            logits = oracle.forward([tok])
    return gen


def teacher_forcing(model, prompt, ref):
    """Feeds prompt + the reference's tokens one at a time; from the last prompt token on, compares
    each position's logits with the reference token that follows (app/llm_real.cpp:292-319)."""
    seq = [int(t) for t in prompt] + [g["id"] for g in ref]
    P, G = len(prompt), len(ref)
    agree = top5_hits = top5_total = 0
    diffs = []
    for p in range(P + G - 1):
        logits = model.forward([seq[p]])
        if p < P - 1:
            continue
        rt = ref[p - (P - 1)]
        ls = log_softmax(logits)
        agree += int(np.argmax(logits)) == rt["id"]
        diffs.append(abs(float(ls[rt["id"]]) - rt["logprob"]))
        kk = len(rt["top"])
        ours = set(int(j) for j in np.argsort(-np.asarray(logits, np.float64), kind="stable")[:kk])
        top5_hits += sum(1 for j in rt["top"] if j in ours)
        top5_total += kk
    return {"agree": agree, "n": G, "mean_abs_dlogp": float(np.mean(diffs)), "max_abs_dlogp": float(np.max(diffs)),
            "top5_overlap": top5_hits / max(1, top5_total)}


def free_run(model, prompt, ref):
    """Greedy from the prompt (prompt fed one token at a time, then the replayed generate): how many
    tokens equal the reference's before the first difference (app/llm_real.cpp:321-334)."""
    model.reset()
    for t in prompt[:-1]:
        model.forward([int(t)])
    model.forward([int(prompt[-1])])
    ours = list(model.generate(len(ref)))
    same = 0
    while same < len(ref) and ours[same] == ref[same]["id"]:
        same += 1
    return same
