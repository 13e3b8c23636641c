/*
 * turns.c -- restatement of the recognizer's word events and of TurnDetector
 * (SVL/stt/mod.rs:283-351, 564-590).
 *
 * TEST INFRASTRUCTURE ONLY (see svl_oracle.h).  Integer and boolean logic:
 *   * Recognizer::step (mod.rs:566-589) pushes the step's VoiceActivity event (when the model has
 *     extra heads), then, when the text token is END_OF_PADDING (0) or PADDING (3) and word
 *     tokens are pending, the Word events of those tokens; a token above PADDING is a pending word
 *     token.  The words' text comes from the tokenizer; a pending run is taken to decode to at
 *     least one word (one Word event or more: TurnDetector treats them alike).
 *   * TurnDetector::update (mod.rs:327-350): a Word sets in_turn; a VoiceActivity counts the
 *     consecutive frames whose probability at index HEAD exceeds the threshold and ends the turn
 *     (returning true, clearing in_turn) once in_turn and the count reaches `frames`.
 */
#include "svl_oracle.h"

enum { END_OF_PADDING = 0, PADDING = 3 };

void svlo_turn_init(svlo_turn* t, float threshold, int frames, int head) {
    t->threshold = threshold;
    t->frames = frames < 1 ? 1 : frames; /* TurnDetector::frames: frames.max(1) */
    t->head = head;
    t->above = 0;
    t->in_turn = 0;
    t->pending = 0;
}

/* TurnDetector::update for a Word event. */
int svlo_turn_word(svlo_turn* t) {
    t->in_turn = 1;
    return 0;
}

/* TurnDetector::update for a VoiceActivity event with `n` pause probabilities. */
int svlo_turn_activity(svlo_turn* t, const float* probs, int n) {
    int pause = t->head >= 0 && t->head < n && probs[t->head] > t->threshold;
    t->above = pause ? t->above + 1 : 0;
    if (t->in_turn && t->above >= (int64_t)t->frames) {
        t->in_turn = 0;
        return 1;
    }
    return 0;
}

/* One recognizer step's events in order, fed to the detector: returns whether they end a turn. */
int svlo_turn_step(svlo_turn* t, uint32_t token, const float* probs, int n) {
    int end = 0;
    if (n > 0) end = svlo_turn_activity(t, probs, n);
    if (token == END_OF_PADDING || token == PADDING) {
        if (t->pending) {
            t->pending = 0;
            svlo_turn_word(t);
        }
    } else if (token > PADDING) {
        t->pending = 1;
    }
    return end;
}
