"""Text in, text out: the token loop of predict_token_by_token
(network_types/transformer/transformer_network.rs:165-313) around
Network.generate, which runs the loop's forward passes and greedy ids on the
device.

What the reference does around the forward pass, restated here:
  - every input is prefixed with "<bos> " (network_components/input.rs:70-72);
  - it is tokenized with the GPT-NeoX tokenizer, special tokens added
    (utils/tokenizer.rs:9-41; tokenize_batch(.., with_eos = false));
  - at most MAX_CONTEXT_WINDOW_SIZE ids are kept, the last ones
    (transformer_network.rs:32, 208-218);
  - each step's greedy id is taken from the last row of sequence 0
    (:258-263) and decoded on its own, special tokens kept
    (utils/tokenizer.rs:43-50);
  - a token that decodes to "<eos>" ends the loop without being appended
    (:285-288); any other token's text is appended to sequence 0's text
    (:291);
  - the loop ends after 21 appended tokens (:293-297).

Only sequence 0 is continued (batch_ids[0].push, :266), so the loop is the
reference's batch-1 path: sequence 0 is generated and the other texts are
returned with their "<bos> " prefix and nothing appended, as the reference
returns them.  The tokenizer is passed in (tokenizers.Tokenizer); the
reference loads it from TOKENIZER_GPT_NEOX_PATH, relative to its crate root.
"""
from __future__ import annotations

import numpy as np

MAX_CONTEXT_WINDOW_SIZE = 512  # transformer_network.rs:32
MAX_NEW_TOKENS = 21            # count_tokens_prediction > 20 ends the loop (:293-297)
EOS_TEXT = "<eos>"             # :285
BOS_PREFIX = "<bos> "          # input.rs:70-72
TOKENIZER_GPT_NEOX_PATH = "src/neural_networks/tokenizers/gtp_neox_tokenizer.json"  # utils/tokenizer.rs:6


def load_tokenizer(path: str):
    """The tokenizer file the reference reads (Tokenizer::from_file)."""
    from tokenizers import Tokenizer

    return Tokenizer.from_file(path)


def predict_token_by_token(net, input_batch, tokenizer):
    """Greedy continuation of input_batch[0] as text.

    Returns (predictions, texts).  `predictions` holds, for every step the
    loop ran, the Re-logits of sequence 0's last row ([vocab] f64).  The
    reference keeps the whole output of the step, which after the first step
    is that one row.  `texts` are the inputs with the "<bos> " prefix,
    sequence 0 extended by the generated tokens' text.
    """
    texts = [BOS_PREFIX + t for t in input_batch]
    if not texts:
        return [], texts
    ids = tokenizer.encode(texts[0], add_special_tokens=True).ids[-MAX_CONTEXT_WINDOW_SIZE:]
    if not ids:
        return [], texts
    prompt = np.asarray([ids], dtype=np.uint32)
    gen, logits = net.generate(prompt, n_new=MAX_NEW_TOKENS, want_logits=True)
    predictions = []
    for k in range(MAX_NEW_TOKENS):
        predictions.append(np.asarray(logits[k][0]))
        token = tokenizer.decode([int(gen[0, k])], skip_special_tokens=False)
        if token == EOS_TEXT:
            break
        texts[0] += token
    return predictions, texts
